"""TurboQuantKVCache on the device (TurboQuant/TurboQuantKVCache.swift,
TQEncoder.swift) against the TurboQuant restatement (oracle.tq_*), which
tests/test_oracle_turboquant.py pins:

  * fromSimpleCache on f16 / bf16 / f32 K/V at D 64, 80 (blockwise
    rotation), 128 and 256 with 1- to 8-bit codes: the encoded records (the
    packed codes and QJL signs, both norms, the exact sink and tail tokens)
    and the decoded unified buffer (its values and its promoted dtype) are
    bit-exact;
  * the window after the compression: appends of 1 and of 300 tokens
    (growth by 256-token steps, the dtype promoted by the concatenation),
    trims inside the window and into the prefix (re-encoding the decoded
    tokens), copy() independence, the state setter;
  * restoreCompressed from the records with and without a window (a window
    of the wrong length empties the cache), restoreFromDecodedKV, and the
    reference's own disk-restore scenario (TQDiskSerializerTests.swift:
    178-219: 96 tokens of [1, 4, *, 16] bf16 at 4/4 bits, then four window
    tokens)."""
import numpy as np
import pytest
import torch

import oracle as O
import vkv
from gpu_util import TORCH, dev, host, rand_bits, values

pytestmark = pytest.mark.gpu

_STATES = {}


def _state(dim, kb, vb, seed=42):
    key = (dim, kb, vb, seed)
    if key not in _STATES:
        _STATES[key] = O.TQState(dim, kb, vb, seed)
    return _STATES[key]


def _simple(k, v, dtype):
    c = vkv.KVCacheSimple()
    c.update(dev(k, dtype), dev(v, dtype))
    return c


def _u32(t):
    return host(t).view(np.uint32).reshape(-1)


def _check_record(got, want, keys, dtype):
    n = int(np.prod(want["shape"]))
    assert got["shape"] == want["shape"] and got["index_bits"] == want["index_bits"]
    assert np.array_equal(_u32(got["indices"]), want["indices"])
    assert np.array_equal(host(got["vec_norms"]).reshape(-1), want["vec_norms"].reshape(-1))
    if keys:
        assert np.array_equal(_u32(got["qjl"]), want["qjl"])
        assert np.array_equal(host(got["res_norms"]).reshape(-1), want["res_norms"].reshape(-1))
    for part in ("sink", "tail"):
        if want[part] is None:
            assert got[part] is None
        else:
            assert np.array_equal(values(got[part], dtype), want[part]), part
    assert n > 0


def _check_decoded(t, want, want_dt):
    dt = {torch.float16: O.F16, torch.float32: O.F32, torch.bfloat16: O.BF16}[t.dtype]
    assert dt == want_dt
    assert np.array_equal(values(t, dt), want)


CASES = [  # dtype, B, H, T, D, key bits, value bits, sink, residual
    (O.BF16, 2, 4, 200, 128, 3, 3, 4, 64),
    (O.F16, 1, 8, 150, 128, 4, 2, 4, 64),
    (O.F32, 2, 2, 90, 64, 2, 4, 0, 0),
    (O.BF16, 1, 2, 300, 256, 3, 3, 4, 16),
    (O.F16, 2, 3, 77, 80, 3, 5, 2, 7),
    (O.BF16, 1, 2, 120, 128, 9, 8, 4, 8),  # 8-bit codes: four to a word
]


@pytest.mark.parametrize("case", CASES, ids=[f"{c[0]}-D{c[4]}-k{c[5]}v{c[6]}" for c in CASES])
def test_from_simple_cache_is_bit_exact(case):
    dtype, B, H, T, D, kb, vb, sink, res = case
    rng = np.random.default_rng(T + D)
    k = rand_bits(rng, (B, H, T, D), dtype, outliers=2)
    v = rand_bits(rng, (B, H, T, D), dtype)
    tq = vkv.TurboQuantKVCache.from_simple_cache(_simple(k, v, dtype), kb, vb, sink, res)
    info = tq.info
    assert info["phase"] == 1 and info["has_encoded"] == 1 and tq.offset == T
    assert info["prefix_tokens"] == T and info["window_tokens"] == 0
    st = _state(D, kb, vb)
    kf, vf = O.to_f32(k, dtype) if dtype != O.F32 else k, O.to_f32(v, dtype) if dtype != O.F32 else v
    ek = O.tq_encode(kf, dtype, st, True, sink, res)
    ev = O.tq_encode(vf, dtype, st, False, sink, res)
    gk, gv = tq.encoded()
    _check_record(gk, ek, True, dtype)
    _check_record(gv, ev, False, dtype)
    dk, dtk = O.tq_decode(ek, st, True)
    dv, dtv = O.tq_decode(ev, st, False)
    sk, sv = tq.state
    _check_decoded(sk, dk, dtk)
    _check_decoded(sv, dv, dtv)
    # the decoded keys stay near the inputs (the codec's own error, largest
    # with 1-bit codes plus the QJL bit)
    rel = np.linalg.norm(dk - kf) / np.linalg.norm(kf)
    assert rel < (0.75 if kb <= 2 else 0.6), rel


def test_no_compressible_middle_gives_an_empty_cache():
    rng = np.random.default_rng(3)
    k = rand_bits(rng, (1, 2, 70, 64), O.BF16)
    tq = vkv.TurboQuantKVCache.from_simple_cache(_simple(k, k, O.BF16), 3, 3)  # 70 - 4 - 64 < 8
    assert tq.offset == 0 and tq.phase == "fill" and tq.state == []
    assert not vkv.TurboQuantKVCache.has_compressible_middle(75)
    assert vkv.TurboQuantKVCache.has_compressible_middle(76)


def _window_case(dtype, sink, res):
    rng = np.random.default_rng(11)
    D, T = 64, 120
    k = rand_bits(rng, (1, 2, T, D), dtype)
    v = rand_bits(rng, (1, 2, T, D), dtype)
    tq = vkv.TurboQuantKVCache.from_simple_cache(_simple(k, v, dtype), 3, 3, sink, res)
    return rng, tq


@pytest.mark.parametrize("dtype,sink,res", [(O.BF16, 4, 64), (O.F16, 4, 64), (O.BF16, 0, 0)])
def test_window_appends_trims_and_copies(dtype, sink, res):
    rng, tq = _window_case(dtype, sink, res)
    base_k, base_v = (x.clone() for x in tq.state)
    udt, cap = base_k.dtype, 120 + 256
    want_k, want_v = [base_k.float().cpu()], [base_v.float().cpu()]
    promote = lambda a, b: a if a == b else torch.float32
    # one token, then 300 (past the 256 free slots: the buffer grows by
    # ceil(300 / 256) steps and the concatenation promotes its dtype)
    for n in (1, 300, 2):
        pos = tq.offset
        if pos + n > cap:
            cap = pos + max(1, (256 + n - 1) // 256) * 256
            udt = promote(udt, torch.bfloat16)
        x = rand_bits(rng, (1, 2, n, 64), O.BF16)
        y = rand_bits(rng, (1, 2, n, 64), O.BF16)
        ok, ov = tq.update(dev(x, O.BF16), dev(y, O.BF16))
        # a window write casts the tokens to the buffer's dtype
        for src, dst in ((x, want_k), (y, want_v)):
            dst.append(torch.from_numpy(O.to_f32(src, O.BF16)).to(udt).float())
        gk, gv = vkv.to_torch(ok), vkv.to_torch(ov)
        assert gk.dtype == udt and gk.shape[2] == tq.offset and tq.capacity == cap
        assert torch.equal(gk.cpu().float()[:, :, -n:], want_k[-1])
        assert torch.equal(gv.cpu().float()[:, :, -n:], want_v[-1])
    full_k = torch.cat(want_k, 2)
    sk, _ = tq.state
    assert torch.equal(sk.cpu().float(), full_k)
    assert tq.offset == 120 + 303 and tq.info["window_tokens"] == 303
    # copy() is independent
    cp = tq.copy()
    x = dev(rand_bits(rng, (1, 2, 1, 64), O.BF16), O.BF16)
    tq.update(x, x)
    assert cp.offset == 423 and tq.offset == 424
    assert torch.equal(cp.state[0].cpu().float(), full_k)
    # trim inside the window: O(1), the prefix kept
    assert tq.trim(10) == 10 and tq.offset == 414 and tq.info["window_tokens"] == 294
    assert torch.equal(tq.state[0].cpu().float(), full_k[:, :, :414])
    # the window written by the old buffer is reused by the next append
    ok, _ = tq.update(x, x)
    assert tq.offset == 415


def test_trim_into_the_prefix_reencodes_the_decoded_tokens():
    rng, tq = _window_case(O.BF16, 4, 16)
    x = dev(rand_bits(rng, (1, 2, 5, 64), O.BF16), O.BF16)
    tq.update(x, x)
    dk, dv = (t.cpu().float().numpy() for t in tq.state)
    assert tq.trim(60) == 60 and tq.offset == 65
    info = tq.info
    assert info["phase"] == 1 and info["prefix_tokens"] == 65 and info["window_tokens"] == 0
    # the reference's slow path: compressFloatKV of the decoded [..<65]
    st = _state(64, 3, 3)
    ek = O.tq_encode(dk[:, :, :65], O.F32, st, True, 4, 16)
    ev = O.tq_encode(dv[:, :, :65], O.F32, st, False, 4, 16)
    gk, gv = tq.encoded()
    _check_record(gk, ek, True, O.F32)
    _check_record(gv, ev, False, O.F32)
    want, dt = O.tq_decode(ek, st, True)
    _check_decoded(tq.state[0], want, dt)
    # trimming everything empties the cache
    assert tq.trim(1000) == 65 and tq.offset == 0 and tq.state == []


def test_state_setter_returns_to_fill():
    rng, tq = _window_case(O.F16, 4, 64)
    k = dev(rand_bits(rng, (1, 2, 33, 64), O.F16), O.F16)
    tq.state = [k, k]
    assert tq.phase == "fill" and tq.offset == 33 and tq.meta_state == [""]
    ok, _ = tq.update(k[:, :, :3], k[:, :, :3])
    assert vkv.to_torch(ok).shape[2] == 36
    assert torch.equal(vkv.to_torch(ok)[:, :, :33].cpu(), k.cpu())


def test_restore_compressed_with_and_without_window():
    rng = np.random.default_rng(21)
    k = rand_bits(rng, (2, 2, 140, 128), O.BF16)
    v = rand_bits(rng, (2, 2, 140, 128), O.BF16)
    src = vkv.TurboQuantKVCache.from_simple_cache(_simple(k, v, O.BF16), 3, 3)
    w = dev(rand_bits(rng, (2, 2, 6, 128), O.BF16), O.BF16)
    src.update(w, w)
    rk, rv = src.encoded()
    wk, wv = src.window_state()
    assert wk.shape[2] == 6 and torch.equal(wk.cpu(), w.cpu().float())
    dst = vkv.TurboQuantKVCache(3, 3)
    dst.restore_compressed(rk, rv, 146, wk, wv)
    assert dst.offset == 146 and dst.info["window_tokens"] == 6
    for a, b in zip(src.state, dst.state):
        assert torch.equal(a.cpu(), b.cpu())
    # no window needed: offset = the encoded tokens
    d2 = vkv.TurboQuantKVCache()
    d2.restore_compressed(rk, rv, 140)
    assert d2.offset == 140 and torch.equal(d2.state[0].cpu(), src.state[0][:, :, :140].cpu())
    # a window of the wrong length, or a missing one, empties the cache
    d3 = vkv.TurboQuantKVCache()
    d3.restore_compressed(rk, rv, 146, wk[:, :, :5].contiguous(), wv[:, :, :5].contiguous())
    assert d3.offset == 0
    d4 = vkv.TurboQuantKVCache()
    d4.restore_compressed(rk, rv, 146)
    assert d4.offset == 0
    # restoreFromDecodedKV: the decoded float seated as the prefix
    d5 = vkv.TurboQuantKVCache()
    sk, sv = src.state
    d5.restore_from_decoded(sk, sv, 146)
    assert d5.offset == 146 and d5.phase == "compressed" and d5.info["has_encoded"] == 0
    assert torch.equal(d5.state[0].cpu(), sk.cpu())


def test_reference_disk_window_scenario():
    """TQDiskSerializerTests.swift:178-219 (shapes and window values)."""
    rng = np.random.default_rng(22)
    k = rand_bits(rng, (1, 4, 96, 16), O.BF16)
    src = vkv.TurboQuantKVCache.from_simple_cache(_simple(k, k, O.BF16), 4, 4, 4)
    wk = torch.full((1, 4, 4, 16), 0.75, dtype=torch.bfloat16, device="cuda")
    wv = torch.full((1, 4, 4, 16), 0.25, dtype=torch.bfloat16, device="cuda")
    src.update(wk, wv)
    assert src.offset == 100 and src.state[0].shape[2] == 100
    w = src.window_state()
    assert w[0].shape[2] == 4 and w[1].shape[2] == 4
    rk, rv = src.encoded()
    assert rk["tail"].shape[2] == 64  # compressedKeys.tailCount == defaultResidualTokens
    dst = vkv.TurboQuantKVCache(4, 4, 4)
    dst.restore_compressed(rk, rv, 100, *w)
    assert dst.offset == 100
    s = dst.state
    assert torch.allclose(s[0][:, :, 96:100].float().cpu(), wk.float().cpu())
    assert torch.allclose(s[1][:, :, 96:100].float().cpu(), wv.float().cpu())


def test_disk_record_with_turboquant_layers(tmp_path):
    """TQDiskSerializer kind 1 (serializeTQLayer :368-429, deserializeTQLayer
    :1244-1346, restoreTQLayer CacheHelpers.swift:1248-1320): a compressed
    layer with a window, a fill-phase layer (kind 2) and a decoded-restored
    layer (kind 2, no encoded payload); read back by the safetensors package
    and restored bit-exact."""
    from safetensors import safe_open
    rng = np.random.default_rng(23)
    k = rand_bits(rng, (1, 4, 96, 16), O.BF16)
    v = rand_bits(rng, (1, 4, 96, 16), O.BF16)
    comp = vkv.TurboQuantKVCache.from_simple_cache(_simple(k, v, O.BF16), 4, 4, 4)
    w = dev(rand_bits(rng, (1, 4, 4, 16), O.BF16), O.BF16)
    comp.update(w, w)
    fill = vkv.TurboQuantKVCache()
    fill.update(dev(k, O.BF16), dev(v, O.BF16))
    dec = vkv.TurboQuantKVCache()
    sk, sv = comp.state
    dec.restore_from_decoded(sk, sv, 100)
    path = str(tmp_path / "tq.safetensors")
    vkv.disk_cache_save(path, [comp, fill, dec])
    with safe_open(path, framework="pt") as f:
        t = {name: f.get_tensor(name) for name in f.keys()}
    assert [t[f"__layer_kind_{i}__"].tolist() for i in range(3)] == [[1], [2], [2]]
    rk, rv = comp.encoded()
    assert t["__tq_0_ck_shape__"].tolist() == rk["shape"] == [1, 4, 28, 16]
    assert t["__tq_0_ck_index_bits__"].tolist() == [3] and t["__tq_0_cv_index_bits__"].tolist() == [4]
    assert t["__tq_0_ck_seed__"].tolist() == [42] and t["__tq_0_offset__"].tolist() == [100]
    assert t["tq_0_ck_indices"].dtype == torch.uint32
    assert np.array_equal(t["tq_0_ck_indices"].view(torch.int32).numpy().view(np.uint32),
                          _u32(rk["indices"]))
    assert t["tq_0_ck_sink"].shape == (1, 4, 4, 16) and t["tq_0_ck_tail"].shape == (1, 4, 64, 16)
    assert t["tq_0_window_keys"].shape == (1, 4, 4, 16)
    back = vkv.disk_cache_load(path)
    assert isinstance(back[0], vkv.TurboQuantKVCache) and back[0].offset == 100
    assert back[0].info["key_bits"] == 4 and back[0].info["window_tokens"] == 4
    for a, b in zip(comp.state, back[0].state):
        assert torch.equal(a.cpu(), b.cpu())
    for src, got in ((fill, back[1]), (dec, back[2])):
        assert isinstance(got, vkv.KVCacheSimple) and got.offset == src.offset
        for a, b in zip(src.state, got.state):
            assert torch.equal(a.cpu(), b.cpu())


def _compressed(rng, dtype, B=1, H=2, T=120, D=64):
    k = rand_bits(rng, (B, H, T, D), dtype)
    v = rand_bits(rng, (B, H, T, D), dtype)
    return vkv.TurboQuantKVCache.from_simple_cache(_simple(k, v, dtype), 3, 3, 4, 16)


@pytest.mark.parametrize("dtype", [O.BF16, O.F16])
def test_compilable_turboquant_follows_the_parent(dtype):
    """CompilableTurboQuantKVCache(from:) then decode steps: the whole unified
    buffers it returns hold, at [0, offset), exactly what the parent cache
    returns for the same steps (bf16 tokens are cast into the f32 unified
    buffer, f16 ones written as they are); the device counters are the
    window position and the offset; attention over the whole buffers with
    its array mask equals attention over the parent's views."""
    rng = np.random.default_rng(7 + dtype)
    D = 64
    tq = _compressed(rng, dtype, D=D)
    c = vkv.CompilableTurboQuantKVCache.from_turboquant(tq)
    assert c.kind == vkv.CACHE_COMPILABLE_TURBOQUANT and c.offset == tq.offset == 120
    win0 = tq.info["window_tokens"]
    for step in range(5):
        k1 = dev(rand_bits(rng, (1, 2, 1, D), dtype), dtype)
        v1 = dev(rand_bits(rng, (1, 2, 1, D), dtype), dtype)
        q = dev(rand_bits(rng, (1, 8, 1, D), dtype), dtype)
        mask = c.make_mask(1)
        ck, cv = (vkv.to_torch(x) for x in c.update(k1, v1))
        tk, tv = (vkv.to_torch(x) for x in tq.update(k1, v1))
        n = tq.offset
        assert c.offset == n == 121 + step
        assert ck.shape[2] >= n and ck.dtype == tk.dtype
        assert torch.equal(ck[:, :, :n], tk) and torch.equal(cv[:, :, :n], tv), step
        m = host(mask)
        assert m.shape == (1, ck.shape[2]) and m[0, :n].all() and not m[0, n:].any()
        inner = c.inner_state()
        assert len(inner) == 4 and inner[0].shape[2] == ck.shape[2]
        assert int(host(vkv.to_torch(inner[2]))[0]) == win0 + step + 1
        assert int(host(vkv.to_torch(inner[3]))[0]) == n
        a = vkv.scaled_dot_product_attention(q, ck.to(q.dtype), cv.to(q.dtype), D ** -0.5,
                                             mask=mask)
        b = vkv.scaled_dot_product_attention(q, tk.to(q.dtype), tv.to(q.dtype), D ** -0.5)
        assert torch.allclose(a.float(), b.float(), atol=2e-2, rtol=2e-2), step


def test_compilable_turboquant_graph_replay():
    """make_mask + update + attention on the compilable cache captured once
    in a HIP graph and replayed with new tokens copied in between: every
    replay equals the same step run eagerly on a twin, and the offset the
    device holds advances by one per replay."""
    dtype, D = O.F16, 64
    rng = np.random.default_rng(77)
    src = _compressed(rng, dtype, D=D)
    cap = vkv.CompilableTurboQuantKVCache.from_turboquant(src)
    twin = vkv.CompilableTurboQuantKVCache.from_turboquant(src)
    kin = torch.zeros((1, 2, 1, D), dtype=torch.float16, device="cuda")
    vin = torch.zeros_like(kin)
    qin = torch.zeros((1, 8, 1, D), dtype=torch.float16, device="cuda")
    out = torch.empty((1, 8, 1, D), dtype=torch.float16, device="cuda")

    def step(cache, o):
        mask = cache.make_mask(1)
        ck, cv = cache.update(kin, vin)
        vkv.scaled_dot_product_attention(qin, ck, cv, D ** -0.5, mask=mask, out=o)

    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        warm = vkv.CompilableTurboQuantKVCache.from_turboquant(src)
        step(warm, torch.empty_like(out))
        cap.make_mask(1)
    torch.cuda.synchronize()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            step(cap, out)
    torch.cuda.synchronize()
    for r in range(4):
        kin.copy_(dev(rand_bits(rng, (1, 2, 1, D), dtype), dtype))
        vin.copy_(dev(rand_bits(rng, (1, 2, 1, D), dtype), dtype))
        qin.copy_(dev(rand_bits(rng, (1, 8, 1, D), dtype), dtype))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        eager = torch.empty_like(out)
        step(twin, eager)
        torch.cuda.synchronize()
        assert torch.equal(out, eager), r
        assert int(host(vkv.to_torch(cap.inner_state()[3]))[0]) == 121 + r


def test_compilable_turboquant_promotion_sanity():
    """CompilableTurboQuantKVCacheTests.swift:108-126: 16 tokens of ones in a
    KVCacheSimple [1, 4, *, 64], fromSimpleCache(keyBits 3, valueBits 3,
    residualTokens 0), then CompilableTurboQuantKVCache(from:): compressed,
    offset 16, and two [1] counters beside the unified buffers."""
    simple = vkv.KVCacheSimple()
    one = torch.ones((1, 4, 1, 64), dtype=torch.float32, device="cuda")
    for _ in range(16):
        simple.update(one, one)
    tq = vkv.TurboQuantKVCache.from_simple_cache(simple, 3, 3, 4, 0)
    assert tq.info["phase"] == 1
    c = vkv.CompilableTurboQuantKVCache.from_turboquant(tq)
    assert c.info["phase"] == 1 and c.offset == 16
    inner = c.inner_state()
    assert len(inner) == 4 and inner[2].shape[0] == 1 and inner[3].shape[0] == 1
    assert int(host(vkv.to_torch(inner[2]))[0]) == 0
    assert int(host(vkv.to_torch(inner[3]))[0]) == 16


def test_compilable_turboquant_past_the_buffers(tmp_path):
    """A compiled decode that runs past the unified buffers: the device
    writes clamp to the buffers (dynamicSliceUpdate), so state is the whole
    buffers (MLX slicing clamps [..<total]), the window is absent
    (serializedWindowState needs the buffers to hold it,
    TurboQuantKVCache.swift:254-258), and a disk save writes the encoded
    record without a window, readable by the safetensors package."""
    from safetensors import safe_open
    rng = np.random.default_rng(91)
    D = 64
    src = _compressed(rng, O.BF16, D=D)
    c = vkv.CompilableTurboQuantKVCache.from_turboquant(src)
    cap = c.inner_state()[0].shape[2]
    steps = cap - c.offset + 1
    k1 = dev(rand_bits(rng, (1, 2, 1, D), O.BF16), O.BF16)
    for _ in range(steps):
        c.update(k1, k1)
    torch.cuda.synchronize()
    assert c.offset == cap + 1
    sk, sv = c.state
    assert sk.shape == (1, 2, cap, D) and sv.shape == (1, 2, cap, D)
    assert c.window_state() is None
    path = str(tmp_path / "past.safetensors")
    vkv.disk_cache_save(path, [c])
    with safe_open(path, framework="pt") as f:
        names = set(f.keys())
        assert f.get_tensor("__tq_0_offset__").tolist() == [cap + 1]
    assert "tq_0_ck_indices" in names and "tq_0_window_keys" not in names


def test_compilable_turboquant_bf16_graph_replay():
    """bf16 tokens into the f32 unified buffers under HIP-graph capture: the
    cast scratch is reserved when the compilable cache is made, so the
    captured update allocates nothing and every replay equals the eager step
    on a twin."""
    dtype, D = O.BF16, 64
    rng = np.random.default_rng(78)
    src = _compressed(rng, dtype, D=D)
    cap = vkv.CompilableTurboQuantKVCache.from_turboquant(src)
    twin = vkv.CompilableTurboQuantKVCache.from_turboquant(src)
    assert vkv.to_torch(cap.inner_state()[0]).dtype == torch.float32
    kin = torch.zeros((1, 2, 1, D), dtype=torch.bfloat16, device="cuda")
    vin = torch.zeros_like(kin)
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    torch.cuda.synchronize()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            cap.update(kin, vin)  # the first compressed update, under capture
    torch.cuda.synchronize()
    for r in range(3):
        kin.copy_(dev(rand_bits(rng, (1, 2, 1, D), dtype), dtype))
        vin.copy_(dev(rand_bits(rng, (1, 2, 1, D), dtype), dtype))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        ck, _ = twin.update(kin, vin)
        torch.cuda.synchronize()
        n = twin.offset
        want = vkv.to_torch(ck)[:, :, n - 1:n]
        full = vkv.to_torch(cap.inner_state()[0])
        assert torch.equal(full[:, :, n - 1:n], want), r
        assert torch.equal(want, kin.float()), r
        assert int(host(vkv.to_torch(cap.inner_state()[3]))[0]) == n
