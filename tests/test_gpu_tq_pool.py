"""TurboQuant caches as pool pages (vkv_turboquant_write_pool): under
batching the reference compresses each slot's cache
(BatchEngine/BatchQuantize.swift:115-125 -> maybeQuantizeKVCache) and
attends the plain K/V its update returns (TurboQuantKVCache.swift:428-500:
the decoded prefix, then the exact window) beside the other slots.  Here a
compressed sequence's K/V are written into pool blocks and attended by
vkv_paged_sdpa with the float (or affine) sequences of the same batch.

Checks: the pool holds exactly the cache's returned K/V (bit-exact through
a gather; cast to the pool dtype with round-to-nearest-even, exact in an
f32 pool; affine pools hold the oracle quantizer's codes of them), a decode
step's new token written after the compression lands beside them, and the
batched attention matches the oracle's SDPA over each sequence's K/V."""
import numpy as np
import pytest
import torch

import oracle as O
import vkv
from gpu_util import TORCH, attn_tol, assert_within, dev, host, rand_bits, values

pytestmark = pytest.mark.gpu


def _tq_slot(rng, H, T, D, B=1, kb=3, vb=3):
    k = rand_bits(rng, (B, H, T, D), O.BF16)
    v = rand_bits(rng, (B, H, T, D), O.BF16)
    simple = vkv.KVCacheSimple()
    simple.update(dev(k, O.BF16), dev(v, O.BF16))
    tq = vkv.TurboQuantKVCache.from_simple_cache(simple, kb, vb)
    assert tq.phase == "compressed" and tq.offset == T
    return tq


def _bits_of(t, dtype):
    """cuda tensor -> host bit patterns in `dtype` (torch casts with RNE)."""
    return host(t.to(TORCH[dtype]).contiguous())


@pytest.mark.parametrize("pool_dtype", [O.BF16, O.F32])
def test_compressed_sequence_joins_a_paged_float_batch(pool_dtype):
    """Two float sequences and a compressed one (200 tokens: 4 sink, 132
    encoded at 3/3 bits, 64 exact) in one pool; then a decode step appends a
    token to every sequence, the compressed one through its cache's update
    and write_pool, the others through paged_append."""
    rng = np.random.default_rng(700 + pool_dtype)
    H, D, bs, Hq = 4, 128, 32, 16
    tq = _tq_slot(rng, H, 200, D)
    lens = [150, 200, 37]
    nblocks = sum((L + bs) // bs + 1 for L in lens) + 2
    pool = vkv.PagedPool(nblocks, bs, 1, H, D, dtype=pool_dtype, bits=0)
    perm = iter(rng.permutation(np.arange(1, nblocks)).tolist())
    tables = [[next(perm) for _ in range((L + 1 + bs - 1) // bs)] for L in lens]
    slot = lambda s, p: tables[s][p // bs] * bs + p % bs
    plain = {s: (rand_bits(rng, (lens[s] + 1, H, D), pool_dtype),
                 rand_bits(rng, (lens[s] + 1, H, D), pool_dtype)) for s in (0, 2)}
    for s, (k, v) in plain.items():
        sl = torch.tensor([slot(s, p) for p in range(lens[s])], dtype=torch.int32, device="cuda")
        pool.append(0, dev(k[:lens[s]], pool_dtype), dev(v[:lens[s]], pool_dtype), sl)
    tq.write_pool(pool, 0, torch.tensor([slot(1, p) for p in range(200)], dtype=torch.int32,
                                        device="cuda"))
    # the decode step: one new token per sequence
    k1 = rand_bits(rng, (1, H, 1, D), O.BF16)
    v1 = rand_bits(rng, (1, H, 1, D), O.BF16)
    tq.update(dev(k1, O.BF16), dev(v1, O.BF16))
    tq.write_pool(pool, 0, torch.tensor([slot(1, 200)], dtype=torch.int32, device="cuda"),
                  first=200, n=1)
    for s, (k, v) in plain.items():
        sl = torch.tensor([slot(s, lens[s])], dtype=torch.int32, device="cuda")
        pool.append(0, dev(k[lens[s]:], pool_dtype), dev(v[lens[s]:], pool_dtype), sl)
    lens = [L + 1 for L in lens]
    tab = np.zeros((3, max(len(t) for t in tables)), np.int32)
    for s, t in enumerate(tables):
        tab[s, :len(t)] = t
    keep = (torch.from_numpy(tab).cuda(), torch.tensor(lens, dtype=torch.int32, device="cuda"))
    view = pool.view(0, keep[0], keep[1], max(lens))
    kd, vd = vkv.paged_gather(view)
    sk, sv = tq.state
    assert sk.shape[2] == 201
    want = {1: (_bits_of(sk[0], pool_dtype), _bits_of(sv[0], pool_dtype))}
    for s, (k, v) in plain.items():
        want[s] = (np.ascontiguousarray(k.transpose(1, 0, 2)),
                   np.ascontiguousarray(v.transpose(1, 0, 2)))
    for s, L in enumerate(lens):
        assert np.array_equal(host(kd[s, :, :L]), want[s][0]), f"keys of seq {s}"
        assert np.array_equal(host(vd[s, :, :L]), want[s][1]), f"values of seq {s}"
    if pool_dtype == O.F32:  # the pool holds update()'s values exactly
        assert sk.dtype == torch.float32
    q = rand_bits(rng, (3, Hq, D), pool_dtype)
    out = values(vkv.paged_attention(dev(q, pool_dtype), view, D ** -0.5), pool_dtype)
    f = (lambda a: O.to_f32(a, pool_dtype)) if pool_dtype != O.F32 else (lambda a: a)
    for s, L in enumerate(lens):
        ref = O.sdpa(f(q[s])[None, :, None], f(want[s][0])[None], f(want[s][1])[None],
                     D ** -0.5)[0, :, 0]
        assert_within(out[s], ref, attn_tol(pool_dtype, ref), f"seq {s}")


@pytest.mark.parametrize("bits", [4, 8])
def test_compressed_batch_rows_into_an_affine_pool(bits):
    """A two-row compressed cache written into a 4/8-bit g64 bf16 pool: the
    codes, scales and biases are the oracle quantizer's of the cast K/V, and
    paged decode attends them as any quantized sequence."""
    rng = np.random.default_rng(800 + bits)
    H, D, bs, T = 2, 128, 32, 150
    tq = _tq_slot(rng, H, T, D, B=2, kb=4, vb=2)
    nb = (T + bs - 1) // bs
    pool = vkv.PagedPool(2 * nb + 3, bs, 1, H, D, dtype=O.BF16, bits=bits)
    perm = rng.permutation(np.arange(1, 2 * nb + 3))
    tables = [perm[:nb], perm[nb:2 * nb]]
    slots = [int(tables[b][p // bs]) * bs + p % bs for b in range(2) for p in range(T)]
    tq.write_pool(pool, 0, torch.tensor(slots, dtype=torch.int32, device="cuda"))
    tab = torch.from_numpy(np.stack(tables).astype(np.int32)).cuda()
    lens = torch.tensor([T, T], dtype=torch.int32, device="cuda")
    view = pool.view(0, tab, lens, T)
    (kq, ks, kb_), (vq, vs, vb_) = vkv.paged_gather_quantized(view)
    sk, sv = tq.state
    for b in range(2):
        for got, src in (((kq, ks, kb_), sk), ((vq, vs, vb_), sv)):
            want = O.quantize(_bits_of(src[b], O.BF16), O.BF16, 64, bits)
            assert np.array_equal(host(got[0][b]), want[0])
            assert np.array_equal(host(got[1][b]), want[1])
            assert np.array_equal(host(got[2][b]), want[2])
    q = rand_bits(rng, (2, 8, D), O.BF16)
    out = values(vkv.paged_attention(dev(q, O.BF16), view, D ** -0.5), O.BF16)
    f = lambda a: O.to_f32(a, O.BF16)
    for b in range(2):
        rk = O.quantize(_bits_of(sk[b], O.BF16), O.BF16, 64, bits)
        rv = O.quantize(_bits_of(sv[b], O.BF16), O.BF16, 64, bits)
        ref, wb = (x[0, :, 0] for x in O.quantized_sdpa(
            f(q[b])[None, :, None], O.BF16, rk[0][None], f(rk[1])[None], f(rk[2])[None],
            rv[0][None], f(rv[1])[None], f(rv[2])[None], D ** -0.5, 64, bits,
            rounding=O.REF_DECODE, bound=True))
        assert_within(out[b], ref, attn_tol(O.BF16, ref) + wb, f"row {b}", wb)


def test_write_pool_refuses_bad_calls():
    rng = np.random.default_rng(900)
    tq = _tq_slot(rng, 2, 120, 64)
    pool = vkv.PagedPool(8, 32, 1, 2, 64, dtype=O.BF16)
    sl = torch.arange(121, dtype=torch.int32, device="cuda")
    with pytest.raises(vkv.VKVError):  # past the cache's offset
        tq.write_pool(pool, 0, sl, first=100, n=21)
    other = vkv.PagedPool(8, 32, 1, 4, 64, dtype=O.BF16)
    with pytest.raises(vkv.VKVError):  # heads differ
        tq.write_pool(other, 0, sl)
    empty = vkv.TurboQuantKVCache()
    with pytest.raises(vkv.VKVError):
        empty.write_pool(pool, 0, sl, n=1)
