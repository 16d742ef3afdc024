"""The router's one-token step over a QuantizedKVCache in one launch
(vkv_attention_with_cache_update: updateQuantized, then
quantizedScaledDotProductAttention, AttentionUtils.swift:94-105,
KVCache.swift:1049-1122, :1909-1997): the matrix-core decode kernel
quantizes the token and stores it into its block before it reads it.

Checked step by step against the two-launch path (the separate_token_write
option: the append launch, then the attention) on a twin cache fed the same
rows: identical output bits, identical cache state (the reference-layout
tuples), no append launch on the one-launch path; the state also equals the
restatement's (oracle/kvcache_ref.py, codes from the oracle quantizer) and
the outputs are within the decode bar of the oracle's quantized SDPA.
Covers capacity growth (the 256-token step), a trim whose next steps
rewrite tokens (the 4-bit value nibbles are merged into words that already
hold other tokens), both bit widths, 64 / 128 / 256 dims, bf16 / f16, and a
batch past 256 rows (launched in slices)."""
import numpy as np
import pytest
import torch

import kvcache_ref as R
import oracle as O
import vkv
from gpu_util import OPTIONS, assert_qclose, dev, host, qref, rand_bits, values

pytestmark = pytest.mark.gpu


def _step(cache, q, k, v, dtype, D, separate, monkeypatch):
    """One router call; returns (output, append launches, decode launches)."""
    monkeypatch.setattr(OPTIONS, "separate_token_write", 1 if separate else 0)
    vkv.kernel_timing(True)
    out = vkv.attention_with_cache_update(dev(q, dtype), dev(k, dtype), dev(v, dtype), cache,
                                          D ** -0.5)
    torch.cuda.synchronize()
    _, n_app = vkv.kernel_timing_read(vkv.TIME_APPEND)
    _, n_dec = vkv.kernel_timing_read(vkv.TIME_DECODE)
    vkv.kernel_timing(False)
    return out, n_app, n_dec


def _same_state(a, b, ref, ctx):
    for i, (x, y) in enumerate(zip(a.state, b.state)):
        hx, hy = host(x), host(y)
        assert np.array_equal(hx, hy), f"{ctx}: state array {i} differs between the paths"
        assert np.array_equal(hx, ref.state[i]), f"{ctx}: state array {i} differs from the restatement"


@pytest.mark.parametrize("bits,D,dtype", [(4, 128, O.BF16), (8, 128, O.BF16), (4, 64, O.F16),
                                          (8, 64, O.BF16), (8, 256, O.BF16), (4, 256, O.F16)])
def test_one_launch_step_equals_two_launches(bits, D, dtype, monkeypatch):
    rng = np.random.default_rng(4100 + bits + D + dtype)
    B, Hkv, Hq = 3, 4, 16
    one, two = vkv.QuantizedKVCache(64, bits), vkv.QuantizedKVCache(64, bits)
    ref = R.QuantizedKVCacheRef(64, bits)
    f = lambda a: O.to_f32(a, dtype)
    print(f"one-launch quantized decode: bits {bits} D {D} dtype {dtype}", flush=True)

    def step(L, ctx):
        q = rand_bits(rng, (B, Hq, L, D), dtype)
        k = rand_bits(rng, (B, Hkv, L, D), dtype, outliers=2)
        v = rand_bits(rng, (B, Hkv, L, D), dtype, outliers=2)
        mask = "causal" if L > 1 else None
        if L > 1:  # a prefill: the two-call path on both
            for c in (one, two):
                vkv.attention_with_cache_update(dev(q, dtype), dev(k, dtype), dev(v, dtype), c,
                                                D ** -0.5, mask=mask)
            ref.update_quantized(k, v, dtype)
            return
        got, n_app, n_dec = _step(one, q, k, v, dtype, D, False, monkeypatch)
        want, m_app, m_dec = _step(two, q, k, v, dtype, D, True, monkeypatch)
        assert (n_app, n_dec) == (0, 1), f"{ctx}: the one-launch step took {n_app} appends"
        assert (m_app, m_dec) == (1, 1), ctx
        assert torch.equal(got, want), f"{ctx}: outputs differ between the paths"
        ref.update_quantized(k, v, dtype)
        kq, ks, kb, vq, vs, vb = ref.state
        r, wb = qref(f(q), dtype, kq, f(ks), f(kb), vq, f(vs), f(vb), D ** -0.5, 64, bits,
                     rounding=O.REF_DECODE)
        assert_qclose(values(got, dtype), r, wb, dtype, ctx)

    step(250, "prefill")
    for i in range(9):  # past 256 tokens: the cache grows on the 7th step
        step(1, f"decode {i}")
        assert one.offset == two.offset == ref.offset
    _same_state(one, two, ref, "after growth")
    for c in (one, two):
        c.trim(6)
    ref.offset -= 6
    for i in range(4):  # rewrite tokens 253.. of words holding others
        step(1, f"after trim {i}")
    assert one.capacity == two.capacity == ref.cap
    _same_state(one, two, ref, "after trim")


def test_one_launch_step_past_256_rows(monkeypatch):
    """300 rows: the decode launches in slices of 256 sequences, each with
    its own rows of the new token."""
    rng = np.random.default_rng(4200)
    dtype, bits, D, B, Hkv, Hq = O.BF16, 4, 64, 300, 1, 4
    one, two = vkv.QuantizedKVCache(64, bits), vkv.QuantizedKVCache(64, bits)
    ref = R.QuantizedKVCacheRef(64, bits)
    print("one-launch quantized decode: 300 rows", flush=True)
    q = rand_bits(rng, (B, Hq, 20, D), dtype)
    k = rand_bits(rng, (B, Hkv, 20, D), dtype)
    v = rand_bits(rng, (B, Hkv, 20, D), dtype)
    for c in (one, two):
        vkv.attention_with_cache_update(dev(q, dtype), dev(k, dtype), dev(v, dtype), c, D ** -0.5,
                                        mask="causal")
    ref.update_quantized(k, v, dtype)
    for i in range(3):
        q = rand_bits(rng, (B, Hq, 1, D), dtype)
        k = rand_bits(rng, (B, Hkv, 1, D), dtype)
        v = rand_bits(rng, (B, Hkv, 1, D), dtype)
        got, n_app, n_dec = _step(one, q, k, v, dtype, D, False, monkeypatch)
        want, _, _ = _step(two, q, k, v, dtype, D, True, monkeypatch)
        assert n_app == 0 and n_dec == 2, (n_app, n_dec)
        assert torch.equal(got, want), f"step {i}"
        ref.update_quantized(k, v, dtype)
    _same_state(one, two, ref, "300 rows")


def test_two_head_groups_keep_the_append_launch(monkeypatch):
    """12 query heads a kv head (two head groups of the decode kernel): the
    step keeps its append launch (two waves would write the token's value
    nibbles) and equals the two-launch path."""
    rng = np.random.default_rng(4300)
    dtype, bits, D, B, Hkv, Hq = O.BF16, 4, 128, 2, 2, 24
    one, two = vkv.QuantizedKVCache(64, bits), vkv.QuantizedKVCache(64, bits)
    print("one-launch quantized decode: two head groups", flush=True)
    q = rand_bits(rng, (B, Hq, 30, D), dtype)
    k = rand_bits(rng, (B, Hkv, 30, D), dtype)
    v = rand_bits(rng, (B, Hkv, 30, D), dtype)
    for c in (one, two):
        vkv.attention_with_cache_update(dev(q, dtype), dev(k, dtype), dev(v, dtype), c, D ** -0.5,
                                        mask="causal")
    for i in range(2):
        q = rand_bits(rng, (B, Hq, 1, D), dtype)
        k = rand_bits(rng, (B, Hkv, 1, D), dtype)
        v = rand_bits(rng, (B, Hkv, 1, D), dtype)
        got, n_app, n_dec = _step(one, q, k, v, dtype, D, False, monkeypatch)
        want, _, _ = _step(two, q, k, v, dtype, D, True, monkeypatch)
        assert (n_app, n_dec) == (1, 1), (n_app, n_dec)
        assert torch.equal(got, want), f"step {i}"
