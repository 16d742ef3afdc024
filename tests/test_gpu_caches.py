"""GPU parity of the per-layer caches (KVCacheSimple, RotatingKVCache,
QuantizedKVCache) through the C ABI against the numpy restatement in
oracle/kvcache_ref.py: returned views, state, metaState, capacities and
masks are bit-exact; attention over the cache is within tolerance of the
CPU oracle."""
import numpy as np
import pytest
import torch

import kvcache_ref as R
import oracle as O
import vkv
from gpu_util import assert_qclose, assert_within, qattn_tol, qref, attn_tol, dev, host, rand_bits, values

pytestmark = pytest.mark.gpu


def view_np(a, dtype=None):
    return host(vkv.to_torch(a))


def test_kvcache_simple_config1():
    """Config 1: fp16, B1, Hkv 8, D 128, seed 0; 512-token prefill then 64
    single-token appends; decode SDPA with 32 query heads after each append.
    Returned K/V and state are bit-exact; capacity follows the step-256 rule
    (KVCache.swift:475-497: 512 -> 768 at the first decode)."""
    dtype = O.F16
    rng = np.random.default_rng(0)
    c = vkv.KVCacheSimple()
    r = R.KVCacheSimpleRef()
    k = rand_bits(rng, (1, 8, 512, 128), dtype)
    v = rand_bits(rng, (1, 8, 512, 128), dtype)
    ok, ov = c.update(dev(k, dtype), dev(v, dtype))
    rk, rv = r.update(k, v)
    assert np.array_equal(view_np(ok), rk) and np.array_equal(view_np(ov), rv)
    assert c.offset == 512 and c.capacity == 512
    for step in range(64):
        k1 = rand_bits(rng, (1, 8, 1, 128), dtype)
        v1 = rand_bits(rng, (1, 8, 1, 128), dtype)
        ok, ov = c.update(dev(k1, dtype), dev(v1, dtype))
        rk, rv = r.update(k1, v1)
        assert c.capacity == r.keys.shape[2]
        if step in (0, 1, 31, 63):
            kk, vv = vkv.to_torch(ok), vkv.to_torch(ov)
            assert np.array_equal(host(kk), rk) and np.array_equal(host(vv), rv)
            q = rand_bits(rng, (1, 32, 1, 128), dtype)
            out = vkv.scaled_dot_product_attention(dev(q, dtype), kk, vv, 128 ** -0.5)
            ref = O.sdpa(O.to_f32(q, dtype), O.to_f32(rk, dtype), O.to_f32(rv, dtype), 128 ** -0.5)
            assert (np.abs(values(out, dtype) - ref) <= attn_tol(dtype, ref)).all()
    assert c.offset == 576 and c.capacity == 768
    st = c.state
    assert np.array_equal(host(st[0]), r.state[0]) and np.array_equal(host(st[1]), r.state[1])
    # trim / copy independence (KVCacheTests.swift:54-141)
    cp = c.copy()
    assert c.trim(10) == 10 and c.offset == 566 and cp.offset == 576
    assert cp.capacity == 576  # copy owns exactly the trimmed state
    k2 = rand_bits(rng, (1, 8, 1, 128), dtype)
    c.update(dev(k2, dtype), dev(k2, dtype))
    assert np.array_equal(host(cp.state[0]), r.state[0])
    assert np.array_equal(host(c.state[0])[:, :, 566], k2[:, :, 0])


@pytest.mark.parametrize("keep", [0, 4])
def test_rotating_cache_matches_restatement(keep):
    dtype = O.BF16
    rng = np.random.default_rng(keep + 1)
    max_size, step = 48, 16
    c = vkv.RotatingKVCache(max_size=max_size, keep=keep, step=step)
    r = R.RotatingKVCacheRef(max_size, keep, step)
    plan = [20] + [1] * 40 + [7] + [1] * 70 + [30] + [1] * 5
    for i, S in enumerate(plan):
        k = rand_bits(rng, (2, 4, S, 64), dtype)
        v = rand_bits(rng, (2, 4, S, 64), dtype)
        mk = c.make_mask(S, window_size=32 if S == 1 else None)
        rmk = r.make_mask(S, window=32 if S == 1 else None)
        if isinstance(rmk, str):
            assert mk == rmk
        else:
            assert np.array_equal(host(mk.to(torch.uint8)).astype(bool), rmk)
        ok, ov = c.update(dev(k, dtype), dev(v, dtype))
        rk, rv = r.update(k, v)
        assert np.array_equal(view_np(ok), rk), i
        assert np.array_equal(view_np(ov), rv), i
        assert c.meta_state == r.meta_state, i
        assert c.offset == r.offset and c.capacity == r.keys.shape[2]
    st = c.state
    assert np.array_equal(host(st[0]), r.state[0])
    tk, tv = c.read_kv()
    rtk, rtv = r.temporally_ordered()
    assert np.array_equal(host(tk), rtk) and np.array_equal(host(tv), rtv)
    # temporal order holds the most recent tokens last (ring invariant)
    cp = c.copy()
    assert cp.meta_state == c.meta_state
    assert c.trim(3) == 3 and r.trim(3) == 3 and c.meta_state == r.meta_state


def test_rotating_physical_growth_with_forced_offset():
    """RotatingKVCachePhysicalGrowthTests.swift:30-74: growth keys on the
    buffer's physical fill, not a large restored offset."""
    dtype = O.BF16
    rng = np.random.default_rng(5)
    c = vkv.RotatingKVCache(max_size=64, keep=0, step=16)
    r = R.RotatingKVCacheRef(64, 0, 16)
    c.meta_state = ["0", "64", "16", "3123", "0"]
    r.offset, r.idx = 3123, 0
    for i in range(80):
        k = rand_bits(rng, (1, 2, 1, 64), dtype)
        ok, ov = c.update(dev(k, dtype), dev(k, dtype))
        rk, _ = r.update(k, k)
        assert np.array_equal(view_np(ok), rk)
        assert c.capacity <= 64 and c.meta_state == r.meta_state


def test_base_make_mask():
    c = vkv.KVCacheSimple()
    assert c.make_mask(1) == "none"
    assert c.make_mask(4) == "causal"
    m = c.make_mask(4, return_array=True)
    assert np.array_equal(host(m.to(torch.uint8)).astype(bool), R.causal_mask(4, 0))
    k = dev(np.zeros((1, 1, 5, 64), np.uint16), O.BF16)
    c.update(k, k)
    m = c.make_mask(3, window_size=4)
    assert np.array_equal(host(m.to(torch.uint8)).astype(bool), R.causal_mask(3, 5, 4))


@pytest.mark.parametrize("bits", [4, 8])
def test_quantized_cache_matches_restatement(bits):
    """QuantizedKVCache.updateQuantized: codes/scales/biases in state are
    bit-exact with the oracle quantizer; metaState and offsets follow the
    reference; decode attention over the cache matches the oracle."""
    dtype = O.BF16
    rng = np.random.default_rng(bits)
    B, Hkv, Hq, D = 2, 8, 32, 128
    c = vkv.QuantizedKVCache(group_size=64, bits=bits)
    r = R.QuantizedKVCacheRef(64, bits)
    for S in [300, 1, 1, 255, 1, 17]:
        k = rand_bits(rng, (B, Hkv, S, D), dtype, outliers=4)
        v = rand_bits(rng, (B, Hkv, S, D), dtype, outliers=4)
        view = c.update_quantized(dev(k, dtype), dev(v, dtype))
        r.update_quantized(k, v, dtype)
        assert c.offset == r.offset and c.capacity == r.cap and c.meta_state == r.meta_state
        if S == 1:
            q = rand_bits(rng, (B, Hq, D), dtype)
            out = vkv.paged_attention(dev(q, dtype), view, D ** -0.5)
            kq, ks, kb, vq, vs, vb = r.state
            f = lambda a: O.to_f32(a, dtype)
            ref, wb = (x[:, :, 0] for x in qref(f(q)[:, :, None], dtype, kq, f(ks), f(kb), vq,
                                                f(vs), f(vb), D ** -0.5, 64, bits))
            assert_qclose(values(out, dtype), ref, wb, dtype, f"S {S} bits {bits}")
    st = c.state
    for got, want in zip(st, r.state):
        assert np.array_equal(host(got).view(want.dtype), want)
    # copy / set_state / toUnquantized
    cp = c.copy()
    for got, want in zip(cp.state, r.state):
        assert np.array_equal(host(got).view(want.dtype), want)
    assert cp.offset == c.offset
    s = c.to_unquantized()
    kd = O.dequantize(r.state[0], r.state[1], r.state[2], dtype, 64, bits)
    assert np.array_equal(host(s.state[0]), kd)
    with pytest.raises(vkv.VKVError, match="updateQuantized"):
        c.update(dev(k, dtype), dev(v, dtype))


def test_to_quantized_from_simple():
    """KVCacheSimple.toQuantized (KVCache.swift:561-581)."""
    dtype = O.BF16
    rng = np.random.default_rng(9)
    s = vkv.KVCacheSimple()
    k = rand_bits(rng, (1, 8, 513, 128), dtype)
    v = rand_bits(rng, (1, 8, 513, 128), dtype)
    s.update(dev(k, dtype), dev(v, dtype))
    q = s.to_quantized(64, 4)
    assert q.offset == 513 and q.capacity == 513
    want = O.quantize(k, dtype, 64, 4)[:3] + O.quantize(v, dtype, 64, 4)[:3]
    for got, w in zip(q.state, want):
        assert np.array_equal(host(got).view(w.dtype), w)
    k1 = rand_bits(rng, (1, 8, 1, 128), dtype)
    q.update_quantized(dev(k1, dtype), dev(k1, dtype))
    assert q.offset == 514 and q.capacity == 513 + 256
