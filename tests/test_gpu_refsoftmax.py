"""Quantized attention with the reference's own arithmetic (the
reference_softmax option, vmlx-swift_amd/csrc/vkv_refattn.hip) and the
group sizes the reference's quantizedScaledDotProductAttention takes
(KVCache.swift:1909-1997; GenerateParameters.kvGroupSize).

The reference path stores the scores in the query dtype, runs
softmax(precise: false) with its AccT = T arithmetic (softmax.h:10-190) and
stores the weights in the dtype before P.V; the oracle restates the same
(REF_DECODE below 16 query tokens, REF_CHUNK from 16 on, whose K/V tiles are
dequantized to the dtype first).  The bar is 2e-2 (1e-4 for f32) + 1 ulp +
the oracle's score-boundary term alone: no weight-rounding term.

Also here: the reference's own quantized-SDPA cases
(Tests/MLXLMTests/KVCacheTests.swift:194-338: D 32, L 4, 8-bit g32 keys
arange(128), identity-row values, causal / bool / additive / fully masked)
on both the default and the reference path."""
import numpy as np
import pytest
import torch

import oracle as O
import vkv
from gpu_util import (OPTIONS, assert_refclose, assert_within, attn_tol, dev, host, qref_flip,
                      rand_bits, values)

pytestmark = pytest.mark.gpu


def tuples(rng, B, Hkv, T, D, dtype, group, bits, outliers=0):
    kx = rand_bits(rng, (B, Hkv, T, D), dtype, outliers=outliers)
    vx = rand_bits(rng, (B, Hkv, T, D), dtype, outliers=outliers)
    kq, ks, kb, _ = O.quantize(kx, dtype, group, bits)
    vq, vs, vb, _ = O.quantize(vx, dtype, group, bits)
    return (kq, ks, kb), (vq, vs, vb)


def run_tuples(q, kt, vt, dtype, scale, group, bits, mask=None):
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a).view(np.int32)).cuda()
    kd = (t(kt[0]), dev(kt[1], dtype), dev(kt[2], dtype))
    vd = (t(vt[0]), dev(vt[1], dtype), dev(vt[2], dtype))
    m = mask
    if isinstance(mask, np.ndarray):
        m = torch.from_numpy(mask).cuda()
    out = vkv.quantized_scaled_dot_product_attention(dev(q, dtype), kd, vd, scale, mask=m,
                                                     group_size=group, bits=bits)
    torch.cuda.synchronize()
    return values(out, dtype)


def oracle_ref(q, kt, vt, dtype, scale, group, bits, mask=None):
    f = lambda a: O.to_f32(a, dtype)
    L = q.shape[2]
    rounding = O.REF_CHUNK if L >= 16 else O.REF_DECODE
    m = mask
    if isinstance(mask, np.ndarray) and mask.dtype != np.bool_:
        m = mask.astype(np.float32)
    return qref_flip(f(q), dtype, kt[0], f(kt[1]), f(kt[2]), vt[0], f(vt[1]), f(vt[2]), scale,
                     group, bits, mask=m, rounding=rounding)


CASES = [  # dtype, B, Hq, Hkv, L, T, D, group, bits, mask, outliers
    (O.BF16, 2, 8, 2, 1, 700, 128, 64, 4, None, 4),
    (O.BF16, 2, 8, 2, 1, 5000, 128, 64, 8, None, 4),      # looped softmax (> 4096 keys)
    (O.BF16, 1, 4, 4, 3, 300, 64, 32, 8, "causal", 0),
    (O.F16, 2, 6, 3, 1, 900, 128, 128, 4, None, 2),
    (O.F16, 1, 8, 2, 5, 257, 96, 32, 4, "bool", 0),
    (O.BF16, 1, 8, 4, 20, 600, 128, 64, 4, "causal", 4),  # the tiled (qmm) path
    (O.BF16, 2, 4, 2, 17, 4500, 128, 128, 8, "causal", 4),
    (O.F32, 1, 4, 2, 2, 333, 64, 64, 8, None, 0),
    (O.BF16, 1, 4, 2, 4, 200, 64, 64, 4, "add_f32", 0),   # f32 mask: fp32 softmax, f32 weights
]


@pytest.mark.parametrize("case", CASES,
                         ids=lambda c: f"dt{c[0]}-L{c[4]}-T{c[5]}-D{c[6]}-g{c[7]}-b{c[8]}-{c[9]}")
def test_reference_softmax_against_oracle(case, monkeypatch):
    dtype, B, Hq, Hkv, L, T, D, group, bits, mask, outl = case
    rng = np.random.default_rng(L * 1000 + T + group + bits)
    print(f"reference softmax: {case}", flush=True)
    q = rand_bits(rng, (B, Hq, L, D), dtype)
    kt, vt = tuples(rng, B, Hkv, T, D, dtype, group, bits, outl)
    m = mask
    if mask == "bool":
        m = rng.random((B, Hq, L, T)) < 0.7
        m[..., 0] = True
    elif mask == "add_f32":
        m = np.where(rng.random((1, 1, L, T)) < 0.8, 0.0, -1e9).astype(np.float32)
    monkeypatch.setattr(OPTIONS, "reference_softmax", 1)
    got = run_tuples(q, kt, vt, dtype, D ** -0.5, group, bits, m)
    ref, fb = oracle_ref(q, kt, vt, dtype, D ** -0.5, group, bits, m)
    assert_refclose(got, ref, fb, dtype, str(case))


@pytest.mark.parametrize("group", [32, 128])
@pytest.mark.parametrize("L", [1, 24])
def test_group_sizes_on_the_default_path(group, L):
    """g32 and g128 caches on the default path (the generic kernel below 16
    query tokens, the gathered matrix-core chunk from 16): within the fp32-
    softmax contract against the oracle (2e-2 + 1 ulp + the weight term)."""
    dtype, B, Hq, Hkv, T, D, bits = O.BF16, 2, 8, 2, 600, 128, 4
    rng = np.random.default_rng(group + L)
    q = rand_bits(rng, (B, Hq, L, D), dtype)
    kt, vt = tuples(rng, B, Hkv, T, D, dtype, group, bits)
    mask = "causal" if L > 1 else None
    got = run_tuples(q, kt, vt, dtype, D ** -0.5, group, bits, mask)
    f = lambda a: O.to_f32(a, dtype)
    ref, wb = O.quantized_sdpa(f(q), dtype, kt[0], f(kt[1]), f(kt[2]), vt[0], f(vt[1]),
                               f(vt[2]), D ** -0.5, group, bits, mask=mask, bound=True,
                               rounding=O.REF_CHUNK if L >= 16 else O.REF_DECODE)
    assert_within(got, ref, attn_tol(dtype, ref) + wb, f"g{group} L{L}", wb)


@pytest.mark.parametrize("group,bits", [(32, 8), (128, 4)])
def test_quantized_cache_group_sizes_through_the_router(group, bits, monkeypatch):
    """QuantizedKVCache(groupSize: 32 / 128) filled and attended through
    attentionWithCacheUpdate (prefill chunk, then decode steps), on the
    default path and with the reference softmax, against the oracle over
    the cache's own state."""
    dtype, B, Hq, Hkv, D = O.BF16, 2, 8, 2, 128
    rng = np.random.default_rng(500 + group)
    for ref_mode in (0, 1):
        monkeypatch.setattr(OPTIONS, "reference_softmax", ref_mode)
        c = vkv.QuantizedKVCache(group_size=group, bits=bits)
        for step, L in enumerate((40, 1, 1)):
            k = rand_bits(rng, (B, Hkv, L, D), dtype)
            v = rand_bits(rng, (B, Hkv, L, D), dtype)
            q = rand_bits(rng, (B, Hq, L, D), dtype)
            mask = "causal" if L > 1 else None
            out = vkv.attention_with_cache_update(dev(q, dtype), dev(k, dtype), dev(v, dtype), c,
                                                  D ** -0.5, mask=mask)
            torch.cuda.synchronize()
            got = values(out, dtype)
            kq, ks, kb, vq, vs, vb = [host(x) for x in c.state]
            f = lambda a: O.to_f32(a, dtype)
            args = (f(q), dtype, kq, f(ks), f(kb), vq, f(vs), f(vb), D ** -0.5, group, bits)
            rnd = O.REF_CHUNK if L >= 16 else O.REF_DECODE
            ctx = f"g{group} step {step} ref {ref_mode}"
            if ref_mode:
                ref, fb = qref_flip(*args, mask=mask, rounding=rnd)
                assert_refclose(got, ref, fb, dtype, ctx)
            else:
                ref, wb = O.quantized_sdpa(*args, mask=mask, rounding=rnd, bound=True)
                assert_within(got, ref, attn_tol(dtype, ref) + wb, ctx, wb)


# ---- Tests/MLXLMTests/KVCacheTests.swift:194-338

def reference_inputs(dtype):
    """makeQuantizedAttentionInputs: queries zeros [1, 1, 4, 32], keys
    arange(128) reshaped [1, 1, 4, 32], values identity rows, the K/V of a
    QuantizedKVCache(groupSize: 32, bits: 8) update."""
    D, L = 32, 4
    q = O.from_f32(np.zeros((1, 1, L, D), np.float32), dtype)
    keys = O.from_f32(np.arange(L * D, dtype=np.float32).reshape(1, 1, L, D), dtype)
    vals = np.zeros((1, 1, L, D), np.float32)
    for i in range(L):
        vals[0, 0, i, i] = 1.0
    vals = O.from_f32(vals, dtype)
    c = vkv.QuantizedKVCache(group_size=32, bits=8)
    c.update_quantized(dev(keys, dtype), dev(vals, dtype))
    kq, ks, kb, vq, vs, vb = c.state
    return q, keys, vals, (kq, ks, kb), (vq, vs, vb)


def additive(mask_bool, dtype):
    """where(mask, 0, finfo.min) in the dtype."""
    lo = -65504.0 if dtype == O.F16 else -3.38953139e38
    return O.from_f32(np.where(mask_bool, 0.0, lo).astype(np.float32), dtype)


TRIL = np.tril(np.ones((4, 4), bool)).reshape(1, 1, 4, 4)


def q_attention(q, kt, vt, dtype, mask):
    m = mask
    if isinstance(mask, np.ndarray):
        m = torch.from_numpy(mask).cuda() if mask.dtype == np.bool_ else dev(mask, dtype)
    out = vkv.quantized_scaled_dot_product_attention(dev(q, dtype), kt, vt, 32 ** -0.5, mask=m,
                                                     group_size=32, bits=8)
    torch.cuda.synchronize()
    return values(out, dtype)


def float_attention(q, k, v, dtype, mask):
    m = mask
    if isinstance(mask, np.ndarray):
        m = torch.from_numpy(mask).cuda() if mask.dtype == np.bool_ else dev(mask, dtype)
    out = vkv.scaled_dot_product_attention(dev(q, dtype), dev(k, dtype), dev(v, dtype),
                                           32 ** -0.5, mask=m)
    torch.cuda.synchronize()
    return values(out, dtype)


def all_close(a, b, rtol=0.05, atol=0.01):
    return np.all(np.abs(a - b) <= atol + rtol * np.abs(b))


@pytest.mark.parametrize("ref_mode", [0, 1])
def test_reference_case_causal_mask(ref_mode, monkeypatch):
    """testQuantizedAttentionCausalMaskMatchesReference (:222-249), f16."""
    monkeypatch.setattr(OPTIONS, "reference_softmax", ref_mode)
    dtype = O.F16
    q, k, v, kt, vt = reference_inputs(dtype)
    out = q_attention(q, kt, vt, dtype, "causal")
    ref = float_attention(q, k, v, dtype, "causal")
    assert np.abs(out[0, 0, 0, 1:4]).max() < 1e-3
    assert all_close(out, ref)


@pytest.mark.parametrize("ref_mode", [0, 1])
@pytest.mark.parametrize("dtype", [O.F16, O.BF16])
def test_reference_case_bool_mask(dtype, ref_mode, monkeypatch):
    """testQuantizedAttentionBooleanArrayMaskMatchesReference (:251-285):
    masked weight at the 8-bit dequantization floor (1e-3 f16, 5e-3 bf16)."""
    monkeypatch.setattr(OPTIONS, "reference_softmax", ref_mode)
    q, k, v, kt, vt = reference_inputs(dtype)
    out = q_attention(q, kt, vt, dtype, TRIL)
    ref = float_attention(q, k, v, dtype, additive(TRIL, dtype))
    tol = 5e-3 if dtype == O.BF16 else 1e-3
    assert np.abs(out[0, 0, 0, 1:4]).max() < tol
    assert all_close(out, ref)


@pytest.mark.parametrize("ref_mode", [0, 1])
def test_reference_case_fully_masked_row_is_finite(ref_mode, monkeypatch):
    """testQuantizedAttentionFullyMaskedRowIsFinite (:287-305)."""
    monkeypatch.setattr(OPTIONS, "reference_softmax", ref_mode)
    dtype = O.F16
    q, k, v, kt, vt = reference_inputs(dtype)
    out = q_attention(q, kt, vt, dtype, np.zeros((1, 1, 4, 4), bool))
    assert np.isfinite(out).all()


@pytest.mark.parametrize("ref_mode", [0, 1])
def test_reference_case_additive_mask(ref_mode, monkeypatch):
    """testQuantizedAttentionAdditiveMaskMatchesReference (:307-338): the
    additive mask in the query dtype on both sides."""
    monkeypatch.setattr(OPTIONS, "reference_softmax", ref_mode)
    dtype = O.F16
    q, k, v, kt, vt = reference_inputs(dtype)
    mask = additive(TRIL, dtype)
    out = q_attention(q, kt, vt, dtype, mask)
    ref = float_attention(q, k, v, dtype, mask)
    assert all_close(out, ref)


def paged_scene(rng, bits, lens, Hkv, D, outliers, bs=32, dtype=O.BF16):
    nblocks = sum((L + bs - 1) // bs for L in lens) + 2
    pool = vkv.PagedPool(nblocks, bs, 1, Hkv, D, dtype=dtype, bits=bits)
    perm = rng.permutation(np.arange(1, nblocks))
    tables, slots, keys, vals, i = [], [], [], [], 0
    for L in lens:
        nb = (L + bs - 1) // bs
        t = [int(b) for b in perm[i:i + nb]]
        i += nb
        tables.append(t)
        slots += [t[p // bs] * bs + p % bs for p in range(L)]
        keys.append(rand_bits(rng, (L, Hkv, D), dtype, outliers=outliers))
        vals.append(rand_bits(rng, (L, Hkv, D), dtype, outliers=outliers))
    pool.append(0, dev(np.concatenate(keys), dtype), dev(np.concatenate(vals), dtype),
                torch.tensor(slots, dtype=torch.int32, device="cuda"))
    width = max(1, max(len(t) for t in tables))
    tab = np.zeros((len(lens), width), np.int32)
    for s, t in enumerate(tables):
        tab[s, :len(t)] = t
    keep = (torch.from_numpy(tab).cuda(), torch.tensor(lens, dtype=torch.int32, device="cuda"))
    view = pool.view(0, keep[0], keep[1], max(lens))
    return pool, view, keys, vals, keep


@pytest.mark.parametrize("bits,D,rep,lens", [
    (4, 128, 4, [4100, 1, 0, 900, 33, 2048, 64, 4097]),
    (8, 128, 4, [6000, 70, 3000]),
    (4, 64, 8, [1500, 31, 250]),
    (8, 256, 2, [2500, 100]),
    (4, 128, 12, [700, 5]),
])
def test_paged_decode_reference_softmax_on_matrix_cores(bits, D, rep, lens, monkeypatch):
    """The reference path of one-token paged decode on matrix cores (bf16
    score rows from the decode kernel, the reference softmax over them, P.V
    from the stored weights, partials summed): mixed lengths across the
    4096-key switch to softmax_looped, empty and one-token sequences, 4 / 8
    query heads per part and head groups, x20 outlier channels; against the
    oracle's REF_DECODE at 2e-2 + 1 ulp + the score-boundary term."""
    dtype, Hkv = O.BF16, 2
    rng = np.random.default_rng(bits * 100 + D + rep)
    print(f"paged reference decode: bits {bits} D {D} rep {rep} lens {lens}", flush=True)
    pool, view, keys, vals, keep = paged_scene(rng, bits, lens, Hkv, D, outliers=4)
    q = rand_bits(rng, (len(lens), Hkv * rep, D), dtype)
    monkeypatch.setattr(OPTIONS, "reference_softmax", 1)
    out = vkv.paged_attention(dev(q, dtype), view, D ** -0.5)
    torch.cuda.synchronize()
    got = values(out, dtype)
    f = lambda a: O.to_f32(a, dtype)
    for s, L in enumerate(lens):
        if L == 0:
            assert (got[s] == 0).all()
            continue
        rk = O.quantize(np.ascontiguousarray(keys[s].transpose(1, 0, 2)), dtype, 64, bits)
        rv = O.quantize(np.ascontiguousarray(vals[s].transpose(1, 0, 2)), dtype, 64, bits)
        ref, fb = (x[0, :, 0] for x in qref_flip(
            f(q[s])[None, :, None], dtype, rk[0][None], f(rk[1])[None], f(rk[2])[None],
            rv[0][None], f(rv[1])[None], f(rv[2])[None], D ** -0.5, 64, bits))
        assert_refclose(got[s], ref, fb, dtype, f"seq {s} len {L}")
