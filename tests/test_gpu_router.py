"""GPU parity of the attention router vkv_attention_with_cache_update
(attentionWithCacheUpdate, AttentionUtils.swift:77-143) against the
oracle: no cache, KVCacheSimple (prefill with a causal mask, decode without
one), QuantizedKVCache (decode through the matrix-core kernel, prefill
through the generic kernel), RotatingKVCache, and CompilableKVCache, whose
array mask the router takes after the update as the reference does."""
import numpy as np
import pytest
import torch

import kvcache_ref as R
import oracle as O
import vkv
from gpu_util import OPTIONS, assert_qclose, assert_within, qattn_tol, qref, attn_tol, dev, host, rand_bits, values

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


@pytest.mark.parametrize("bits", [4, 8])
def test_update_quantized_then_quantized_attention(bits):
    """A model that calls updateQuantized and then
    quantizedScaledDotProductAttention itself (GPTOSS.swift:239-248,
    MiMoV2Flash.swift:36-45): the paged view updateQuantized returns is
    attended over directly for any query length and mask, without a state
    gather; against the reference-arithmetic oracle."""
    dtype, D, Hkv, Hq = O.BF16, 128, 2, 8
    rng = np.random.default_rng(30 + bits)
    c, r = vkv.QuantizedKVCache(64, bits), R.QuantizedKVCacheRef(64, bits)
    f = lambda a: O.to_f32(a, dtype)
    for L, mask in [(20, "causal"), (1, None), (5, "causal"), (1, "bool"), (3, None)]:
        q = rand_bits(rng, (2, Hq, L, D), dtype)
        k = rand_bits(rng, (2, Hkv, L, D), dtype)
        v = rand_bits(rng, (2, Hkv, L, D), dtype)
        view = c.update_quantized(dev(k, dtype), dev(v, dtype))
        r.update_quantized(k, v, dtype)
        T = r.offset
        m_dev = m_ref = mask
        if mask == "bool":
            m = rng.random((2, Hq, L, T)) > 0.3
            m_dev, m_ref = torch.from_numpy(m).cuda(), m
        out = vkv.quantized_paged_attention(dev(q, dtype), view, D ** -0.5, mask=m_dev)
        kq, ks, kb, vq, vs, vb = r.state
        ref, wb = qref(f(q), dtype, kq, f(ks), f(kb), vq, f(vs), f(vb), D ** -0.5, 64,
                       bits, mask=m_ref, rounding=O.REF_CHUNK if L >= 16 else O.REF_DECODE)
        assert_qclose(values(out, dtype), ref, wb, dtype, f"L {L} mask {mask}")


def test_quantized_attention_over_pool_view_chunks():
    """A chunk of 4 query tokens per sequence over a paged pool with mixed
    lengths (continuous batching): causal per sequence (query l of a
    sequence of T tokens sees keys t <= T - 4 + l)."""
    dtype, bits, D, Hkv, Hq, bs, L = O.BF16, 4, 128, 2, 8, 32, 4
    rng = np.random.default_rng(40)
    lens = [37, 300, 4, 129]
    nb = sum((n + bs - 1) // bs for n in lens) + 1
    pool = vkv.PagedPool(nb, bs, 1, Hkv, D, dtype=vkv.BF16, bits=bits)
    perm = rng.permutation(np.arange(1, nb))
    tables, slots, keys, vals, i = [], [], [], [], 0
    for n in lens:
        t = [int(x) for x in perm[i:i + (n + bs - 1) // bs]]
        i += len(t)
        tables.append(t)
        slots += [t[p // bs] * bs + p % bs for p in range(n)]
        keys.append(rand_bits(rng, (n, Hkv, D), dtype))
        vals.append(rand_bits(rng, (n, Hkv, D), dtype))
    pool.append(0, dev(np.concatenate(keys), dtype), dev(np.concatenate(vals), dtype),
                torch.tensor(slots, dtype=torch.int32, device="cuda"))
    tab = np.zeros((len(lens), max(len(t) for t in tables)), np.int32)
    for s, t in enumerate(tables):
        tab[s, :len(t)] = t
    tab_d = torch.from_numpy(tab).cuda()
    len_d = torch.tensor(lens, dtype=torch.int32, device="cuda")
    view = pool.view(0, tab_d, len_d, max(lens))
    q = rand_bits(rng, (len(lens), Hq, L, D), dtype)
    out = values(vkv.quantized_paged_attention(dev(q, dtype), view, D ** -0.5, mask="causal"),
                 dtype)
    f = lambda a: O.to_f32(a, dtype)
    for s, n in enumerate(lens):
        rk = O.quantize(np.ascontiguousarray(keys[s].transpose(1, 0, 2)), dtype, 64, bits)
        rv = O.quantize(np.ascontiguousarray(vals[s].transpose(1, 0, 2)), dtype, 64, bits)
        ref, wb = (x[0] for x in qref(f(q[s])[None], dtype, rk[0][None], f(rk[1])[None],
                                      f(rk[2])[None], rv[0][None], f(rv[1])[None], f(rv[2])[None],
                                      D ** -0.5, 64, bits, mask="causal"))
        assert_qclose(out[s], ref, wb, dtype, f"sequence {s} (length {n})")


@pytest.mark.parametrize("bits,D,window", [(4, 128, 0), (8, 128, 0), (8, 256, 0), (4, 128, 64)])
def test_quantized_chunk_over_ragged_pool_view_on_matrix_cores(bits, D, window, monkeypatch):
    """A 20-token chunk per sequence over a paged pool with ragged lengths
    (the continuous-batching prefill step): 16 or more query tokens take the
    gather + matrix-core path with per-sequence lengths.  A sequence shorter
    than the chunk leaves its first queries without a visible key, which the
    reference's where(mask, s, finfo.min) turns into uniform weights (the
    mean of V); against the oracle with the multi-token arithmetic
    (REF_CHUNK) and against the generic kernel."""
    dtype, Hkv, Hq, bs, L = O.BF16, 2, 8, 32, 20
    rng = np.random.default_rng(41 + bits + D)
    lens = [300, 37, 5, 129, 20, 1000]
    nb = sum((n + bs - 1) // bs for n in lens) + 1
    pool = vkv.PagedPool(nb, bs, 1, Hkv, D, dtype=vkv.BF16, bits=bits)
    perm = rng.permutation(np.arange(1, nb))
    tables, slots, keys, vals, i = [], [], [], [], 0
    for n in lens:
        t = [int(x) for x in perm[i:i + (n + bs - 1) // bs]]
        i += len(t)
        tables.append(t)
        slots += [t[p // bs] * bs + p % bs for p in range(n)]
        keys.append(rand_bits(rng, (n, Hkv, D), dtype))
        vals.append(rand_bits(rng, (n, Hkv, D), dtype))
    pool.append(0, dev(np.concatenate(keys), dtype), dev(np.concatenate(vals), dtype),
                torch.tensor(slots, dtype=torch.int32, device="cuda"))
    tab = np.zeros((len(lens), max(len(t) for t in tables)), np.int32)
    for s, t in enumerate(tables):
        tab[s, :len(t)] = t
    view = pool.view(0, torch.from_numpy(tab).cuda(),
                     torch.tensor(lens, dtype=torch.int32, device="cuda"), max(lens))
    q = rand_bits(rng, (len(lens), Hq, L, D), dtype)
    run = lambda: values(vkv.quantized_paged_attention(dev(q, dtype), view, D ** -0.5,
                                                       mask="causal"), dtype)
    # window > 0: K/V gathered 64 tokens at a time, so the shorter rows have
    # windows past their end
    monkeypatch.setattr(OPTIONS, "gather_tokens", window)
    out = run()
    monkeypatch.setattr(OPTIONS, "generic_attention", 1)
    gen = run()
    f = lambda a: O.to_f32(a, dtype)
    for s, n in enumerate(lens):
        rk = O.quantize(np.ascontiguousarray(keys[s].transpose(1, 0, 2)), dtype, 64, bits)
        rv = O.quantize(np.ascontiguousarray(vals[s].transpose(1, 0, 2)), dtype, 64, bits)
        ref, wb = (x[0] for x in qref(f(q[s])[None], dtype, rk[0][None], f(rk[1])[None],
                                      f(rk[2])[None], rv[0][None], f(rv[1])[None], f(rv[2])[None],
                                      D ** -0.5, 64, bits, mask="causal", rounding=O.REF_CHUNK))
        assert_within(out[s], ref, qattn_tol(dtype, ref, wb), f"sequence {s} (length {n})", wb)
        assert_within(out[s], gen[s], attn_tol(dtype, ref) + 2 * wb, f"generic, sequence {s}", wb)
