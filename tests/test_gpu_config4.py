"""The Gemma-style rotating workload at its shapes: 16 query / 8 kv heads
of 256 dims, batch 4, bf16 K/V ~ N(0,1).

Sliding-window layer: a RotatingKVCache(maxSize: 1024, keep: 0)
(Gemma3Text.swift:412-415) driven through attentionWithCacheUpdate
(AttentionUtils.swift:77-143): a 700-token causal prefill chunk, then
single-token decode steps until the ring has wrapped twice (idx returns to
slot 0 twice, KVCache.swift:755-769).  Offset and metaState are checked
against the restatement every step, the cache's arrays bit-exact after the
second wrap, and the attention output against the oracle's float SDPA
(fp32 softmax, MLXFast semantics) at the prefill, around each wrap and
every 128th step.

Global layer: an 8-bit g64 QuantizedKVCache at the full 32768-token
context: one prefill update of 32767 tokens, then one decode token through
the router; the state (codes, scales, biases) is bit-exact with the oracle
quantizer and the decode output matches the oracle with the reference's
arithmetic."""
import numpy as np
import pytest

import kvcache_ref as R
import oracle as O
import vkv
from gpu_util import assert_qclose, assert_within, attn_tol, dev, host, qref, rand_bits, values

pytestmark = pytest.mark.gpu

B, HQ, HKV, D = 4, 16, 8, 256


def test_config4_sliding_window_layer_two_wraps():
    dtype, M = O.BF16, 1024
    rng = np.random.default_rng(400)
    c, r = vkv.RotatingKVCache(M, keep=0), R.RotatingKVCacheRef(M, 0)
    f = lambda a: O.to_f32(a, dtype)
    wraps, step, prev_idx = 0, 0, 0
    checks = 0
    while wraps < 2:
        S = 700 if step == 0 else 1
        q = rand_bits(rng, (B, HQ, S, D), dtype)
        k = rand_bits(rng, (B, HKV, S, D), dtype)
        v = rand_bits(rng, (B, HKV, S, D), dtype)
        # the model's mask, made before the update (Gemma3Text.swift: the
        # sliding layers ask makeMask(n, windowSize: slidingWindow)):
        # "causal" for the prefill chunk, none for a decode token
        mask = r.make_mask(S, window=M)
        assert mask in ("causal", "none")
        mask = None if mask == "none" else mask
        out = vkv.attention_with_cache_update(dev(q, dtype), dev(k, dtype), dev(v, dtype), c,
                                              D ** -0.5, mask=mask)
        rk, rv = r.update(k, v)
        assert c.offset == r.offset and c.meta_state == r.meta_state, step
        idx = int(r.meta_state[4])
        if idx < prev_idx:
            wraps += 1
            print(f"config 4 window: wrap {wraps} at step {step} (offset {r.offset})", flush=True)
        near_wrap = idx <= 1 or idx >= M - 1
        if step == 0 or near_wrap or step % 128 == 0:
            ref = O.sdpa(f(q), f(rk), f(rv), D ** -0.5, mask)
            assert_within(values(out, dtype), ref, attn_tol(dtype, ref), f"step {step}")
            checks += 1
        prev_idx = idx
        step += 1
    # the cache's own arrays equal the restatement's after two wraps
    st = c.state
    assert np.array_equal(host(st[0]), r.state[0]) and np.array_equal(host(st[1]), r.state[1])
    assert checks >= 10


def test_config4_global_layer_8bit_full_context():
    dtype, bits, T = O.BF16, 8, 32768
    rng = np.random.default_rng(401)
    print(f"config 4 global: prefill {T - 1} tokens", flush=True)
    c = vkv.QuantizedKVCache(group_size=64, bits=bits)
    k0 = rand_bits(rng, (B, HKV, T - 1, D), dtype)
    v0 = rand_bits(rng, (B, HKV, T - 1, D), dtype)
    c.update_quantized(dev(k0, dtype), dev(v0, dtype))
    k1 = rand_bits(rng, (B, HKV, 1, D), dtype)
    v1 = rand_bits(rng, (B, HKV, 1, D), dtype)
    q = rand_bits(rng, (B, HQ, 1, D), dtype)
    out = vkv.attention_with_cache_update(dev(q, dtype), dev(k1, dtype), dev(v1, dtype), c,
                                          D ** -0.5)
    assert c.offset == T
    kx = np.concatenate([k0, k1], axis=2)
    vx = np.concatenate([v0, v1], axis=2)
    del k0, v0
    st = c.state
    refs = []
    for which, x in ((0, kx), (1, vx)):
        rq, rs, rb, _ = O.quantize(x, dtype, 64, bits)
        assert np.array_equal(host(st[3 * which]), rq), which
        assert np.array_equal(host(st[3 * which + 1]).view(rs.dtype), rs), which
        assert np.array_equal(host(st[3 * which + 2]).view(rb.dtype), rb), which
        refs.append((rq, rs, rb))
    print("config 4 global: state bit-exact; checking attention", flush=True)
    f = lambda a: O.to_f32(a, dtype)
    (kq, ks, kb), (vq, vs, vb) = refs
    ref, wb = qref(f(q), dtype, kq, f(ks), f(kb), vq, f(vs), f(vb), D ** -0.5, 64, bits)
    assert_qclose(values(out, dtype), ref, wb, dtype, "global layer")
