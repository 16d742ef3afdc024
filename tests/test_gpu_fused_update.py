"""A router decode step over a KVCacheSimple or RotatingKVCache
(attentionWithCacheUpdate, AttentionUtils.swift:106-142: update, then
MLXFast SDPA over the returned views) writes the new token inside the float
decode kernel, which reads it from the caller's rows and stores it into the
cache as it goes (one launch fewer a step).  Against a twin cache updated
by vkv_cache_update and attended by vkv_sdpa: the cache states are
bit-exact and the outputs equal (same kernel, same split) -- including the
paths that hand the write back to a copy (the generic kernel, a head dim the
decode kernel does not take, a growth step)."""
import numpy as np
import pytest
import torch

import oracle as O
import vkv
from gpu_util import OPTIONS, dev, host, rand_bits

pytestmark = pytest.mark.gpu


def twin_steps(make, dtype, B, H, Hq, D, pre, steps, rng, sinks=False):
    a, b = make(), make()
    k0 = dev(rand_bits(rng, (B, H, pre, D), dtype), dtype)
    v0 = dev(rand_bits(rng, (B, H, pre, D), dtype), dtype)
    a.update(k0, v0)
    b.update(k0, v0)
    sk = dev(rand_bits(rng, (Hq,), dtype), dtype) if sinks else None
    for i in range(steps):
        k1 = dev(rand_bits(rng, (B, H, 1, D), dtype), dtype)
        v1 = dev(rand_bits(rng, (B, H, 1, D), dtype), dtype)
        q = dev(rand_bits(rng, (B, Hq, 1, D), dtype), dtype)
        got = vkv.attention_with_cache_update(q, k1, v1, a, D ** -0.5, sinks=sk)
        ck, cv = b.update(k1, v1)
        m = b.make_mask(1, return_array=True)  # as the router asks for it
        mask = m if isinstance(m, torch.Tensor) else None
        want = vkv.scaled_dot_product_attention(q, ck, cv, D ** -0.5, sinks=sk, mask=mask)
        torch.cuda.synchronize()
        assert np.array_equal(host(got), host(want)), f"step {i}"
        assert a.offset == b.offset
        for x, y in zip(a.state, b.state):
            assert np.array_equal(host(x), host(y)), f"state after step {i}"


@pytest.mark.parametrize("dtype,D,rep,B", [(O.BF16, 128, 4, 1), (O.F16, 256, 2, 2),
                                           (O.F32, 64, 8, 1), (O.BF16, 80, 2, 1)])
def test_simple_cache_decode_writes_the_token_in_the_kernel(dtype, D, rep, B):
    """KVCacheSimple: steps inside the 256-token capacity, then one that
    grows it (the token after a growth copy); D 80 takes the generic
    kernel, which gets the copy first."""
    rng = np.random.default_rng(D + rep + dtype)
    print(f"fused update, simple: dtype {dtype} D {D} rep {rep} B {B}", flush=True)
    twin_steps(vkv.KVCacheSimple, dtype, B, 2, 2 * rep, D, 250, 9, rng)


@pytest.mark.parametrize("sinks", [False, True])
def test_rotating_cache_decode_writes_the_token_in_the_kernel(sinks):
    """RotatingKVCache(maxSize 64): past the first wrap, in place at the ring
    index, with the ring's array mask when the window is smaller."""
    rng = np.random.default_rng(77 + sinks)
    print(f"fused update, rotating: sinks {sinks}", flush=True)
    twin_steps(lambda: vkv.RotatingKVCache(64), O.BF16, 2, 4, 8, 128, 60, 12, rng, sinks)


def test_generic_option_takes_the_copy(monkeypatch):
    monkeypatch.setattr(OPTIONS, "generic_attention", 1)
    rng = np.random.default_rng(5)
    twin_steps(vkv.KVCacheSimple, O.BF16, 1, 2, 8, 128, 100, 3, rng)
