"""GPU parity of the attention router vkv_attention_with_cache_update
(attentionWithCacheUpdate, AttentionUtils.swift:77-143) against the
oracle: no cache, KVCacheSimple (prefill with a causal mask, decode without
one), QuantizedKVCache (decode through the matrix-core kernel, prefill
through the generic kernel), RotatingKVCache, and CompilableKVCache, whose
array mask the router takes after the update as the reference does."""
import numpy as np
import pytest

import kvcache_ref as R
import oracle as O
import vkv
from gpu_util import assert_qclose, assert_within, qattn_tol, qref, attn_tol, dev, host, rand_bits, values

pytestmark = pytest.mark.gpu


def close(got, ref, dtype):
    return (np.abs(values(got, dtype) - ref) <= attn_tol(dtype, ref)).all()


def test_router_without_cache():
    dtype, D = O.BF16, 64
    rng = np.random.default_rng(1)
    q = rand_bits(rng, (2, 8, 3, D), dtype)
    k = rand_bits(rng, (2, 2, 3, D), dtype)
    v = rand_bits(rng, (2, 2, 3, D), dtype)
    out = vkv.attention_with_cache_update(dev(q, dtype), dev(k, dtype), dev(v, dtype), None,
                                          D ** -0.5, mask="causal")
    f = lambda a: O.to_f32(a, dtype)
    assert close(out, O.sdpa(f(q), f(k), f(v), D ** -0.5, "causal"), dtype)


def test_router_simple_cache_prefill_then_decode():
    dtype, D = O.F16, 128
    rng = np.random.default_rng(2)
    c, r = vkv.KVCacheSimple(), R.KVCacheSimpleRef()
    f = lambda a: O.to_f32(a, dtype)
    for L, mask in [(16, "causal"), (1, None), (1, None), (5, "causal")]:
        q = rand_bits(rng, (1, 8, L, D), dtype)
        k = rand_bits(rng, (1, 2, L, D), dtype)
        v = rand_bits(rng, (1, 2, L, D), dtype)
        out = vkv.attention_with_cache_update(dev(q, dtype), dev(k, dtype), dev(v, dtype), c,
                                              D ** -0.5, mask=mask)
        rk, rv = r.update(k, v)
        assert c.offset == r.offset
        assert close(out, O.sdpa(f(q), f(rk), f(rv), D ** -0.5, mask), dtype), L


@pytest.mark.parametrize("bits", [4, 8])
def test_router_quantized_cache(bits):
    dtype, D, Hkv, Hq = O.BF16, 128, 4, 16
    rng = np.random.default_rng(3 + bits)
    c, r = vkv.QuantizedKVCache(64, bits), R.QuantizedKVCacheRef(64, bits)
    f = lambda a: O.to_f32(a, dtype)
    for L, mask in [(40, "causal"), (1, None), (1, None), (3, "causal")]:
        q = rand_bits(rng, (2, Hq, L, D), dtype)
        k = rand_bits(rng, (2, Hkv, L, D), dtype)
        v = rand_bits(rng, (2, Hkv, L, D), dtype)
        out = vkv.attention_with_cache_update(dev(q, dtype), dev(k, dtype), dev(v, dtype), c,
                                              D ** -0.5, mask=mask)
        r.update_quantized(k, v, dtype)
        kq, ks, kb, vq, vs, vb = r.state
        # 16+ query tokens run on the matrix (qmm) path, fewer on the vector path
        ref, wb = qref(f(q), dtype, kq, f(ks), f(kb), vq, f(vs), f(vb), D ** -0.5, 64,
                       bits, mask=mask, rounding=O.REF_CHUNK if L >= 16 else O.REF_DECODE)
        assert c.offset == r.offset
        assert_qclose(values(out, dtype), ref, wb, dtype, f"L {L}")


def test_router_rotating_cache_decode():
    dtype, D = O.BF16, 64
    rng = np.random.default_rng(4)
    c, r = vkv.RotatingKVCache(16), R.RotatingKVCacheRef(16)
    f = lambda a: O.to_f32(a, dtype)
    for step in range(24):
        q = rand_bits(rng, (1, 4, 1, D), dtype)
        k = rand_bits(rng, (1, 2, 1, D), dtype)
        v = rand_bits(rng, (1, 2, 1, D), dtype)
        out = vkv.attention_with_cache_update(dev(q, dtype), dev(k, dtype), dev(v, dtype), c,
                                              D ** -0.5)
        rk, rv = r.update(k, v)
        assert close(out, O.sdpa(f(q), f(rk), f(rv), D ** -0.5), dtype), step


def test_router_compilable_cache_takes_cache_mask():
    """The router asks the cache for a mask after the update
    (AttentionUtils.swift:106-142), so a fixed-buffer cache's row covers
    positions 0 .. offset (post-update) of its buffer."""
    dtype, D, M = O.BF16, 64, 64
    rng = np.random.default_rng(5)
    c = vkv.CompilableKVCache(max_length=M)
    r = R.CompilableKVCacheRef(M)
    f = lambda a: O.to_f32(a, dtype)
    for step, L in enumerate([7, 1, 1, 1]):
        q = rand_bits(rng, (1, 4, L, D), dtype)
        k = rand_bits(rng, (1, 2, L, D), dtype)
        v = rand_bits(rng, (1, 2, L, D), dtype)
        out = vkv.attention_with_cache_update(dev(q, dtype), dev(k, dtype), dev(v, dtype), c,
                                              D ** -0.5)
        rk, rv = r.update(k, v)
        ref = O.sdpa(f(q), f(rk), f(rv), D ** -0.5, r.make_mask(L))
        assert c.offset == r.offset
        assert close(out, ref, dtype), step
