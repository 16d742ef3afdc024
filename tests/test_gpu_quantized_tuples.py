"""QuantizedKVCache.updateQuantized's return value
(vkv_cache_update_quantized_tuples, KVCache.swift:1049-1122): the keys' and
values' (wq, scales, biases) trimmed to offset, in the reference layout,
checked bit-exact against the restatement (oracle/kvcache_ref.py, whose
codes come from the oracle quantizer) over a prefill that crosses the
256-token step, decode steps, a chunk, a trim followed by an update that
rewrites the trimmed tokens, and a state setter; beside them the paged view
of the same cache stays usable (its state equals the tuples)."""
import numpy as np
import pytest

import kvcache_ref as R
import oracle as O
import vkv
from gpu_util import dev, host, rand_bits

pytestmark = pytest.mark.gpu


def _check(got, ref, cap, ctx):
    gk, gv = got
    want = ref.state
    for i, a in enumerate(list(gk) + list(gv)):
        assert a.shape[2] == ref.offset and a.strides[1] == cap * a.shape[3], ctx
        assert np.array_equal(host(vkv.to_torch(a)), want[i]), f"{ctx}: array {i}"


@pytest.mark.parametrize("bits,group,dtype", [(4, 64, O.BF16), (8, 64, O.F16), (4, 32, O.BF16),
                                              (8, 128, O.BF16)])
def test_update_quantized_returns_the_reference_tuples(bits, group, dtype):
    rng = np.random.default_rng(1300 + bits + group + dtype)
    B, H, D = 2, 4, 128
    c = vkv.QuantizedKVCache(group_size=group, bits=bits)
    r = R.QuantizedKVCacheRef(group, bits)

    def step(S, ctx):
        k = rand_bits(rng, (B, H, S, D), dtype, outliers=2)
        v = rand_bits(rng, (B, H, S, D), dtype, outliers=2)
        got = c.update_quantized_tuples(dev(k, dtype), dev(v, dtype))
        r.update_quantized(k, v, dtype)
        assert c.offset == r.offset and c.capacity == r.cap, ctx
        _check(got, r, r.cap, ctx)

    print(f"tuples: bits {bits} group {group} dtype {dtype}", flush=True)
    step(300, "prefill 300")       # capacity 512
    for i in range(3):
        step(1, f"decode {i}")
    step(50, "chunk 50")
    c.trim(20)                     # the next update rewrites tokens 334..
    r.offset -= 20
    step(5, "after trim")
    step(200, "growth")            # 339 + 200 > 512: capacity grows
    # the paged update of the same cache, then tuples again
    k = rand_bits(rng, (B, H, 1, D), dtype)
    v = rand_bits(rng, (B, H, 1, D), dtype)
    c.update_quantized(dev(k, dtype), dev(v, dtype))
    r.update_quantized(k, v, dtype)
    step(1, "after a paged update")
    for got, want in zip(c.state, r.state):
        assert np.array_equal(host(got), want)


def test_tuples_after_the_state_setter():
    """set_state replaces every token: the next tuples come from the new
    state, not from what the cache held before."""
    rng = np.random.default_rng(1400)
    B, H, D, dtype, bits = 1, 2, 64, O.BF16, 4
    a = vkv.QuantizedKVCache(group_size=64, bits=bits)
    b = vkv.QuantizedKVCache(group_size=64, bits=bits)
    ra = R.QuantizedKVCacheRef(64, bits)
    for cache, ref in ((a, ra), (b, None)):
        k = rand_bits(rng, (B, H, 40, D), dtype)
        v = rand_bits(rng, (B, H, 40, D), dtype)
        cache.update_quantized_tuples(dev(k, dtype), dev(v, dtype))
        if ref is not None:
            ref.update_quantized(k, v, dtype)
    b.state = a.state
    b.meta_state = a.meta_state
    k = rand_bits(rng, (B, H, 1, D), dtype)
    v = rand_bits(rng, (B, H, 1, D), dtype)
    got = b.update_quantized_tuples(dev(k, dtype), dev(v, dtype))
    ra.update_quantized(k, v, dtype)
    _check(got, ra, b.capacity, "after set_state")


def test_tuples_need_a_quantized_cache():
    c = vkv.KVCacheSimple()
    x = dev(rand_bits(np.random.default_rng(1), (1, 1, 2, 64), O.BF16), O.BF16)
    with pytest.raises(vkv.VKVError):
        vkv._chk(vkv.lib().vkv_cache_update_quantized_tuples(
            c._h, vkv.C.byref(vkv.arr(x)), vkv.C.byref(vkv.arr(x)), vkv.stream_ptr(),
            (vkv.Array * 6)()))
