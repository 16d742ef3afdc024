"""Paged decode over caches quantized with group 128 on the matrix-core
kernel (its group-128 mode: quantizedScaledDotProductAttention,
KVCache.swift:1909-1997, with GenerateParameters.kvGroupSize 128,
Evaluate.swift:109-112), where each scale / bias pair serves two of the
kernel's 64-dim groups.  Mixed sequence lengths (an empty and a one-token
sequence among them), 4 / 8 bits, 128 / 256 dims, bf16 / f16, 1 to 8 query
heads a kv head, ×20 outlier channels: against the oracle's quantized SDPA
over the same codes (the fp32-softmax contract, 2e-2 + 1 ulp + the
reference's weight-rounding term) and against the generic kernel; the
kernel timing counts show the matrix-core kernel ran.  Group 128 with the
reference softmax keeps the generic reference path."""
import numpy as np
import pytest
import torch

import oracle as O
import vkv
from gpu_util import OPTIONS, assert_qclose, attn_tol, assert_within, dev, qref, rand_bits, values

pytestmark = pytest.mark.gpu


def scene(rng, bits, group, lens, Hkv, D, dtype, bs=32):
    """A pool of the sequences' K/V (random blocks), its view with the real
    lengths (0 included) and the per-sequence rows [L, Hkv, D]."""
    stored = [max(L, 1) for L in lens]
    nblocks = sum((L + bs - 1) // bs for L in stored) + 2
    pool = vkv.PagedPool(nblocks, bs, 1, Hkv, D, dtype=dtype, bits=bits, group_size=group)
    perm = rng.permutation(np.arange(1, nblocks))
    tables, slots, keys, vals, i = [], [], [], [], 0
    for L in stored:
        nb = (L + bs - 1) // bs
        t = [int(b) for b in perm[i:i + nb]]
        i += nb
        tables.append(t)
        slots += [t[p // bs] * bs + p % bs for p in range(L)]
        keys.append(rand_bits(rng, (L, Hkv, D), dtype, outliers=2))
        vals.append(rand_bits(rng, (L, Hkv, D), dtype, outliers=2))
    pool.append(0, dev(np.concatenate(keys), dtype), dev(np.concatenate(vals), dtype),
                torch.tensor(slots, dtype=torch.int32, device="cuda"))
    tab = np.zeros((len(lens), max(len(t) for t in tables)), np.int32)
    for s, t in enumerate(tables):
        tab[s, :len(t)] = t
    tab_dev = torch.from_numpy(tab).cuda()
    len_dev = torch.tensor(lens, dtype=torch.int32, device="cuda")
    view = pool.view(0, tab_dev, len_dev, max(stored))
    return pool, view, keys, vals, (tab_dev, len_dev)


def decode(q, view, D, timed=False):
    if timed:
        vkv.kernel_timing(True)
    out = vkv.paged_attention(q, view, D ** -0.5)
    torch.cuda.synchronize()
    n = 0
    if timed:
        _, n = vkv.kernel_timing_read(vkv.TIME_DECODE)
        vkv.kernel_timing(False)
    return out, n


@pytest.mark.parametrize("bits,D,dtype,rep", [(4, 128, O.BF16, 4), (8, 128, O.F16, 1),
                                              (4, 256, O.F16, 2), (8, 256, O.BF16, 8),
                                              (4, 128, O.F16, 8), (8, 128, O.BF16, 3)])
def test_group128_decode_on_matrix_cores(bits, D, dtype, rep):
    rng = np.random.default_rng(8100 + bits + D + dtype + rep)
    Hkv, group = 2, 128
    lens = [700, 1, 0, 2100, 64, 333]
    print(f"group-128 decode: bits {bits} D {D} dtype {dtype} rep {rep}", flush=True)
    pool, view, keys, vals, keep = scene(rng, bits, group, lens, Hkv, D, dtype)
    q = rand_bits(rng, (len(lens), Hkv * rep, D), dtype)
    out, n_dec = decode(dev(q, dtype), view, D, timed=True)
    assert n_dec == 1, "the matrix-core decode did not run"
    got = values(out, dtype)
    f = lambda a: O.to_f32(a, dtype)
    for s, L in enumerate(lens):
        if L == 0:
            assert not got[s].any(), "an empty sequence yields zeros"
            continue
        rk = O.quantize(np.ascontiguousarray(keys[s][:L].transpose(1, 0, 2)), dtype, group, bits)
        rv = O.quantize(np.ascontiguousarray(vals[s][:L].transpose(1, 0, 2)), dtype, group, bits)
        ref, wb = (x[0, :, 0] for x in qref(f(q[s])[None, :, None], dtype, rk[0][None],
                                            f(rk[1])[None], f(rk[2])[None], rv[0][None],
                                            f(rv[1])[None], f(rv[2])[None], D ** -0.5, group,
                                            bits))
        assert_qclose(got[s], ref, wb, dtype, f"seq {s} (len {L})")


def test_group128_matches_the_generic_kernel(monkeypatch):
    """The same call on the generic VALU kernel (the generic_attention
    option): within 2e-2 of each other plus an ulp of the output dtype for
    each side's own rounding (different fp32 orders, the same codes)."""
    rng = np.random.default_rng(8200)
    dtype, bits, D, Hkv, rep = O.BF16, 4, 128, 8, 4
    lens = [1500, 37, 4000, 900]
    print("group-128 decode against the generic kernel", flush=True)
    pool, view, keys, vals, keep = scene(rng, bits, 128, lens, Hkv, D, dtype)
    q = dev(rand_bits(rng, (len(lens), Hkv * rep, D), dtype), dtype)
    mc, n_dec = decode(q, view, D, timed=True)
    assert n_dec == 1
    monkeypatch.setattr(OPTIONS, "generic_attention", 1)
    gen, n_gen = decode(q, view, D, timed=True)
    assert n_gen == 0, "the generic option still ran the matrix-core decode"
    a, b = values(mc, dtype), values(gen, dtype)
    assert_within(a, b, attn_tol(dtype, b) + 2.0 ** -8 * np.abs(b),
                  "matrix cores against the generic kernel")


def test_group128_reference_softmax_keeps_the_generic_path(monkeypatch):
    """The matrix-core reference path stores group-64 score rows only: with
    the reference softmax a group-128 decode runs the generic reference
    path (no matrix-core decode launch) and still meets its bar."""
    rng = np.random.default_rng(8300)
    dtype, bits, D, Hkv, rep = O.BF16, 8, 128, 2, 4
    lens = [300, 5]
    print("group-128 decode with the reference softmax", flush=True)
    pool, view, keys, vals, keep = scene(rng, bits, 128, lens, Hkv, D, dtype)
    q = rand_bits(rng, (len(lens), Hkv * rep, D), dtype)
    monkeypatch.setattr(OPTIONS, "reference_softmax", 1)
    out, n_dec = decode(dev(q, dtype), view, D, timed=True)
    assert n_dec == 0
    got = values(out, dtype)
    f = lambda a: O.to_f32(a, dtype)
    for s, L in enumerate(lens):
        rk = O.quantize(np.ascontiguousarray(keys[s].transpose(1, 0, 2)), dtype, 128, bits)
        rv = O.quantize(np.ascontiguousarray(vals[s].transpose(1, 0, 2)), dtype, 128, bits)
        ref, fb = (x[0, :, 0] for x in O.quantized_sdpa(
            f(q[s])[None, :, None], dtype, rk[0][None], f(rk[1])[None], f(rk[2])[None],
            rv[0][None], f(rv[1])[None], f(rv[2])[None], D ** -0.5, 128, bits,
            rounding=O.REF_DECODE, flip=True))
        assert_within(got[s], ref, attn_tol(dtype, ref) + fb, f"seq {s}", fb)
