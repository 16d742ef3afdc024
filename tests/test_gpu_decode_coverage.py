"""The matrix-core paged decode (qdecode_kernel) on the caches it used to
hand to the generic kernel: f16 caches (f16 score MFMAs on f16 key
operands, bf16 P.V, f16 output) and contexts past 126,976 tokens (more than
32 partials per (sequence, head pair), merged 4 at a time past the first
32).  Each case checks that the matrix-core kernel ran (the library's
kernel timing counts its launches) and its output against the oracle's
quantized SDPA with the reference's rounding (REF_DECODE), at 2e-2 + 1 ulp
+ the oracle's bound for the single-pass fp32 softmax.
(QuantizedKVCache.quantizedScaledDotProductAttention, KVCache.swift:
1909-1997, takes any float dtype and length; sdpa_vector.h:179-394 splits
any length.)"""
import numpy as np
import pytest
import torch

import oracle as O
import vkv
from gpu_util import assert_within, attn_tol, dev, qref, rand_bits, values

pytestmark = pytest.mark.gpu


def scene(rng, dtype, bits, lens, Hkv, D, outliers=0, bs=32):
    nblocks = sum((L + bs - 1) // bs for L in lens) + 2
    pool = vkv.PagedPool(nblocks, bs, 1, Hkv, D, dtype=dtype, bits=bits)
    perm = rng.permutation(np.arange(1, nblocks))
    tables, slots, keys, vals, i = [], [], [], [], 0
    for L in lens:
        nb = (L + bs - 1) // bs
        t = perm[i:i + nb].astype(np.int64)
        i += nb
        tables.append(t)
        pos = np.arange(L)
        slots.append(t[pos // bs] * bs + pos % bs)
        keys.append(rand_bits(rng, (L, Hkv, D), dtype, outliers=outliers))
        vals.append(rand_bits(rng, (L, Hkv, D), dtype, outliers=outliers))
    pool.append(0, dev(np.concatenate(keys), dtype), dev(np.concatenate(vals), dtype),
                torch.from_numpy(np.concatenate(slots).astype(np.int32)).cuda())
    width = max(len(t) for t in tables)
    tab = np.zeros((len(lens), width), np.int32)
    for s, t in enumerate(tables):
        tab[s, :len(t)] = t
    keep = (torch.from_numpy(tab).cuda(), torch.tensor(lens, dtype=torch.int32, device="cuda"))
    return pool, pool.view(0, keep[0], keep[1], max(lens)), keys, vals, keep


def run_and_check(rng, dtype, bits, lens, Hkv, rep, D, outliers):
    pool, view, keys, vals, keep = scene(rng, dtype, bits, lens, Hkv, D, outliers)
    q = rand_bits(rng, (len(lens), Hkv * rep, D), dtype)
    vkv.kernel_timing(True)
    out = vkv.paged_attention(dev(q, dtype), view, D ** -0.5)
    torch.cuda.synchronize()
    _, launches = vkv.kernel_timing_read(vkv.TIME_DECODE)
    vkv.kernel_timing(False)
    assert launches == 1, "the matrix-core decode kernel did not run"
    got = values(out, dtype)
    f = lambda a: O.to_f32(a, dtype)
    for s, L in enumerate(lens):
        rk = O.quantize(np.ascontiguousarray(keys[s].transpose(1, 0, 2)), dtype, 64, bits)
        rv = O.quantize(np.ascontiguousarray(vals[s].transpose(1, 0, 2)), dtype, 64, bits)
        ref, wb = (x[0, :, 0] for x in qref(
            f(q[s])[None, :, None], dtype, rk[0][None], f(rk[1])[None], f(rk[2])[None],
            rv[0][None], f(rv[1])[None], f(rv[2])[None], D ** -0.5, 64, bits))
        assert_within(got[s], ref, attn_tol(dtype, ref) + wb, f"seq {s} len {L}", wb)


@pytest.mark.parametrize("bits,D,rep,lens", [
    (4, 128, 4, [4097, 700, 33, 1]),
    (8, 128, 4, [3000, 64]),
    (4, 64, 8, [1500, 250]),
    (8, 256, 2, [2100, 90]),
    (4, 128, 12, [900, 31]),
])
def test_f16_cache_on_matrix_cores(bits, D, rep, lens):
    """An f16 QuantizedKVCache's pages (config-2 shapes and others, x20
    outlier channels): queries and scores in f16 as the reference stores
    them, f16 output."""
    rng = np.random.default_rng(9000 + bits * 10 + D + rep)
    print(f"f16 decode: bits {bits} D {D} rep {rep} lens {lens}", flush=True)
    run_and_check(rng, O.F16, bits, lens, 2, rep, D, outliers=4)


def test_config2_shape_f16_on_matrix_cores():
    """Config 2's shape in f16: B 8 x 4097 tokens, 8 / 32 heads x 128,
    4-bit g64, x20 outliers."""
    rng = np.random.default_rng(9100)
    print("f16 decode: config-2 shape", flush=True)
    run_and_check(rng, O.F16, 4, [4097] * 8, 8, 4, 128, outliers=4)


def test_long_context_131072_tokens():
    """One sequence of 131,072 tokens (8 / 32 heads x 128, 4-bit), past the
    126,976 tokens that 32 partials per pair covered, beside a short one."""
    rng = np.random.default_rng(9200)
    print("long context: 131072 + 100 tokens", flush=True)
    run_and_check(rng, O.BF16, 4, [131072, 100], 8, 4, 128, outliers=0)


def test_long_context_among_many_short_sequences():
    """The merge inside the decode launch past 32 partials: 255 sequences of
    40 tokens beside one of 131,072 give 2048 (sequence, head pair)s, so the
    launch averages at most 4 partials a pair and merges inside, while the
    long pair has about 33 partials (more than the 32 of one merge step);
    the short pairs' few partials merge inside the same launch."""
    rng = np.random.default_rng(9250)
    lens = [40] * 120 + [131072] + [40] * 135
    print(f"long context among {len(lens)} sequences", flush=True)
    run_and_check(rng, O.BF16, 4, lens, 8, 4, 128, outliers=0)


def test_long_context_reference_softmax(monkeypatch):
    """The reference-arithmetic decode (score rows, the looped reference
    softmax, P.V from stored weights) over 131,072 tokens: more than 32
    plain-sum partials per pair."""
    from gpu_util import OPTIONS, assert_refclose, qref_flip
    monkeypatch.setattr(OPTIONS, "reference_softmax", 1)
    rng = np.random.default_rng(9300)
    dtype, bits, Hkv, rep, D = O.BF16, 4, 2, 4, 128
    lens = [131072, 5]
    print(f"long context, reference softmax: {lens}", flush=True)
    pool, view, keys, vals, keep = scene(rng, dtype, bits, lens, Hkv, D)
    q = rand_bits(rng, (len(lens), Hkv * rep, D), dtype)
    out = vkv.paged_attention(dev(q, dtype), view, D ** -0.5)
    torch.cuda.synchronize()
    got = values(out, dtype)
    f = lambda a: O.to_f32(a, dtype)
    for s, L in enumerate(lens):
        rk = O.quantize(np.ascontiguousarray(keys[s].transpose(1, 0, 2)), dtype, 64, bits)
        rv = O.quantize(np.ascontiguousarray(vals[s].transpose(1, 0, 2)), dtype, 64, bits)
        ref, fb = (x[0, :, 0] for x in qref_flip(
            f(q[s])[None, :, None], dtype, rk[0][None], f(rk[1])[None], f(rk[2])[None],
            rv[0][None], f(rv[1])[None], f(rv[2])[None], D ** -0.5, 64, bits))
        assert_refclose(got[s], ref, fb, dtype, f"seq {s} len {L}")
