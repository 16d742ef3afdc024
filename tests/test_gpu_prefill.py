"""GPU parity of multi-query attention (L >= 2 query tokens: chunked prefill)
over dense bf16 / f16 K/V with no or a causal mask, the matrix-core path of
vkv_sdpa (vkv_prefill.hip), against the oracle's SDPA and against the
generic kernel (the generic_attention option): GQA groups of 1, 4 and 8, key
counts that are not multiples of the 32-token tile, query counts that are
not multiples of the 256-row block, several key splits, strided slices of
cache buffers and two batch rows; head dims 64, 128 and 256 (at 256 the two
waves of a SIMD split the output dims).  Quantized K/V (a QuantizedKVCache's
paged chunks, or reference-layout code/scale/bias arrays) with 16+ query
tokens take the same kernel after a gather to bf16 rows."""
import numpy as np
import pytest
import torch

import oracle as O
import vkv
from gpu_util import OPTIONS, assert_qclose, assert_within, qattn_tol, qref, attn_tol, dev, rand_bits, values

pytestmark = pytest.mark.gpu


def run_case(rng, dtype, B, Hq, Hkv, L, T, mask, cap=None, monkeypatch=None, scale=None, D=128):
    scale = D ** -0.5 if scale is None else scale
    q = rand_bits(rng, (B, Hq, L, D), dtype)
    k = rand_bits(rng, (B, Hkv, T, D), dtype)
    v = rand_bits(rng, (B, Hkv, T, D), dtype)
    if cap:  # slices of larger (cache-like) buffers: token stride D, head stride cap * D
        kb = torch.zeros((B, Hkv, cap, D), dtype=dev(k, dtype).dtype, device="cuda")
        vb = torch.zeros_like(kb)
        kb[:, :, :T] = dev(k, dtype)
        vb[:, :, :T] = dev(v, dtype)
        kd, vd = kb[:, :, :T], vb[:, :, :T]
    else:
        kd, vd = dev(k, dtype), dev(v, dtype)
    got = values(vkv.scaled_dot_product_attention(dev(q, dtype), kd, vd, scale, mask=mask), dtype)
    f = lambda a: O.to_f32(a, dtype)
    ref = O.sdpa(f(q), f(k), f(v), scale, mask=mask)
    bad = np.abs(got - ref) > attn_tol(dtype, ref)
    assert not bad.any(), (np.abs(got - ref).max(), np.argwhere(bad)[:4])
    if monkeypatch is not None:
        monkeypatch.setattr(OPTIONS, "generic_attention", 1)
        gen = values(vkv.scaled_dot_product_attention(dev(q, dtype), kd, vd, scale, mask=mask),
                     dtype)
        monkeypatch.setattr(OPTIONS, "generic_attention", 0)
        assert (np.abs(got - gen) <= attn_tol(dtype, ref)).all()


@pytest.mark.parametrize("dtype", [O.BF16, O.F16])
@pytest.mark.parametrize("mask", [None, "causal"])
@pytest.mark.parametrize("Hq,Hkv", [(32, 8), (8, 8), (16, 2)])
def test_prefill_matches_oracle(dtype, mask, Hq, Hkv, monkeypatch):
    rng = np.random.default_rng(dtype * 100 + Hq + Hkv + (mask == "causal"))
    run_case(rng, dtype, 1, Hq, Hkv, 70, 301, mask, monkeypatch=monkeypatch)


@pytest.mark.parametrize("L,T", [(2, 2), (2, 33), (31, 31), (64, 1000), (300, 700)])
def test_prefill_lengths_causal(L, T):
    rng = np.random.default_rng(L * 7 + T)
    run_case(rng, O.BF16, 1, 32, 8, L, T, "causal")


def test_prefill_no_mask_long_keys_many_splits():
    # few query rows and many keys: several key splits merged
    rng = np.random.default_rng(5)
    run_case(rng, O.BF16, 1, 8, 8, 4, 4133, None)


def test_prefill_chunk_over_cache_slice_two_rows():
    # a 512-token chunk at the end of a 1500-token context, cache buffers of
    # capacity 1792, two batch rows
    rng = np.random.default_rng(9)
    run_case(rng, O.BF16, 2, 8, 2, 512, 1500, "causal", cap=1792)


def test_prefill_large_scores_rescale():
    # scores that grow along the keys exercise the running-max rescale
    rng = np.random.default_rng(13)
    run_case(rng, O.BF16, 1, 16, 4, 40, 600, "causal", scale=0.5)


@pytest.mark.parametrize("dtype", [O.BF16, O.F16])
@pytest.mark.parametrize("mask", [None, "causal"])
@pytest.mark.parametrize("D", [64, 256])
def test_prefill_head_dims(dtype, mask, D, monkeypatch):
    # Gemma-style 16 / 8 heads at 256 dims; 64 dims
    rng = np.random.default_rng(dtype * 10 + D + (mask == "causal"))
    run_case(rng, dtype, 1, 16, 8, 70, 301, mask, monkeypatch=monkeypatch, D=D)


@pytest.mark.parametrize("D", [64, 256])
@pytest.mark.parametrize("L,T", [(2, 33), (300, 700)])
def test_prefill_head_dims_lengths(D, L, T):
    # two batch rows of cache-buffer slices; short and long chunks
    rng = np.random.default_rng(D + L + T)
    run_case(rng, O.BF16, 2, 8, 2, L, T, "causal", cap=T + 40, D=D)


def test_prefill_256_long_keys_many_splits():
    rng = np.random.default_rng(17)
    run_case(rng, O.BF16, 1, 16, 8, 6, 3000, None, D=256)


def quantized_chunk(rng, bits, outliers, T0=300, L=64, Hkv=8, D=128, rep=4):
    """An L-token causal chunk through the router over a QuantizedKVCache
    holding a T0-token prefix (GQA rep): returns the output, the chunk's
    inputs and the whole (prefix + chunk) K/V."""
    dtype, Hq = O.BF16, rep * Hkv
    k0, v0 = (rand_bits(rng, (1, Hkv, T0, D), dtype, outliers=outliers) for _ in range(2))
    k1, v1 = (rand_bits(rng, (1, Hkv, L, D), dtype, outliers=outliers) for _ in range(2))
    q = rand_bits(rng, (1, Hq, L, D), dtype)
    c = vkv.QuantizedKVCache(group_size=64, bits=bits)
    c.update_quantized(dev(k0, dtype), dev(v0, dtype))

    def step():
        out = vkv.attention_with_cache_update(dev(q, dtype), dev(k1, dtype), dev(v1, dtype), c,
                                              D ** -0.5, mask="causal")
        assert c.trim(L) == L
        return values(out, dtype)

    return step, q, np.concatenate([k0, k1], axis=2), np.concatenate([v0, v1], axis=2)


@pytest.mark.parametrize("bits", [4, 8])
def test_quantized_cache_chunk(bits, monkeypatch):
    """Against the oracle's quantized SDPA on the same codes, and against the
    generic path (which keeps the dequantized values unrounded)."""
    dtype, D = O.BF16, 128
    step, q, kx, vx = quantized_chunk(np.random.default_rng(bits), bits, 0)
    got = step()
    kq, ks, kb, _ = O.quantize(kx, dtype, 64, bits)
    vq, vs, vb, _ = O.quantize(vx, dtype, 64, bits)
    f = lambda a: O.to_f32(a, dtype)
    ref, wb = qref(f(q), dtype, kq, f(ks), f(kb), vq, f(vs), f(vb), D ** -0.5, 64, bits,
                   mask="causal", rounding=O.REF_CHUNK)
    tol = qattn_tol(dtype, ref, wb)
    assert_within(got, ref, tol, "oracle", wb)
    monkeypatch.setattr(OPTIONS, "generic_attention", 1)
    gen = step()
    assert_within(got, gen, attn_tol(dtype, ref) + 2 * wb, "generic", wb)


@pytest.mark.parametrize("bits,window", [(4, 96), (8, 32), (4, 160)])
def test_quantized_cache_chunk_key_windows(bits, window, monkeypatch):
    """The chunk's K/V gathered one key window at a time (the gather_tokens
    option; by default a window's copy is at most 256 MiB): against the
    oracle and against the single-window result (the same arithmetic, only
    the split merge groups differently)."""
    dtype, D = O.BF16, 128
    step, q, kx, vx = quantized_chunk(np.random.default_rng(70 + bits + window), bits, 0, T0=500,
                                      L=64)
    whole = step()
    monkeypatch.setattr(OPTIONS, "gather_tokens", window)
    got = step()
    kq, ks, kb, _ = O.quantize(kx, dtype, 64, bits)
    vq, vs, vb, _ = O.quantize(vx, dtype, 64, bits)
    f = lambda a: O.to_f32(a, dtype)
    ref, wb = qref(f(q), dtype, kq, f(ks), f(kb), vq, f(vs), f(vb), D ** -0.5, 64, bits,
                   mask="causal", rounding=O.REF_CHUNK)
    assert_qclose(got, ref, wb, dtype, f"window {window}")
    assert_within(got, whole, attn_tol(dtype, ref), "one window")


@pytest.mark.parametrize("D,bits,rep", [(256, 8, 2), (64, 4, 4)])
def test_quantized_cache_chunk_head_dims(D, bits, rep, monkeypatch):
    """A chunk over a QuantizedKVCache at 256 dims (config 4's 8-bit global
    layer, 16 / 8 heads) and at 64 dims, against the oracle and the generic
    path."""
    dtype = O.BF16
    step, q, kx, vx = quantized_chunk(np.random.default_rng(D + bits), bits, 0, T0=500, L=96,
                                      Hkv=8, D=D, rep=rep)
    got = step()
    kq, ks, kb, _ = O.quantize(kx, dtype, 64, bits)
    vq, vs, vb, _ = O.quantize(vx, dtype, 64, bits)
    f = lambda a: O.to_f32(a, dtype)
    ref, wb = qref(f(q), dtype, kq, f(ks), f(kb), vq, f(vs), f(vb), D ** -0.5, 64, bits,
                   mask="causal", rounding=O.REF_CHUNK)
    assert_qclose(got, ref, wb, dtype, f"D {D}")
    monkeypatch.setattr(OPTIONS, "generic_attention", 1)
    gen = step()
    assert_within(got, gen, attn_tol(dtype, ref) + 2 * wb, "generic", wb)


@pytest.mark.parametrize("ref_mode", [1, 0], ids=["reference_softmax", "fp32_softmax"])
@pytest.mark.parametrize("bits", [4, 8])
def test_quantized_cache_chunk_outlier_channels(bits, ref_mode, monkeypatch):
    """Config-2 data (4 channels per head scaled x20), a 512-token chunk
    over a 4096-token cache: against the reference's matrix-path rounding
    (affine_qmm dequantizes K/V tiles to bf16, quantized.h:568-576,
    :686-713; scores and weights stored in bf16, KVCache.swift:1945-1982).
    With the reference softmax the bar holds the score-boundary term alone;
    the single-pass matrix-core kernel (fp32 softmax) adds the weight term."""
    dtype, D = O.BF16, 128
    monkeypatch.setattr(OPTIONS, "reference_softmax", ref_mode)
    step, q, kx, vx = quantized_chunk(np.random.default_rng(10 + bits), bits, 4, T0=3584,
                                      L=512, Hkv=2)
    got = step()
    kq, ks, kb, _ = O.quantize(kx, dtype, 64, bits)
    vq, vs, vb, _ = O.quantize(vx, dtype, 64, bits)
    f = lambda a: O.to_f32(a, dtype)
    ref, wb, fb = O.quantized_sdpa(f(q), dtype, kq, f(ks), f(kb), vq, f(vs), f(vb), D ** -0.5,
                                   64, bits, mask="causal", rounding=O.REF_CHUNK, bound=True,
                                   flip=True)
    if ref_mode:
        assert_within(got, ref, attn_tol(dtype, ref) + fb, f"bits {bits} reference softmax", fb)
    else:
        assert_qclose(got, ref, wb, dtype, f"bits {bits}")


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("L,mask", [(32, "causal"), (48, None)])
def test_quantized_sdpa_reference_layout_chunk(bits, L, mask, monkeypatch):
    """Stateless quantized SDPA over reference-layout (codes, scales, biases)
    arrays with 16+ query tokens: gathered to bf16 rows, then the
    matrix-core kernel; against the oracle's quantized SDPA and against the
    generic path."""
    dtype, B, Hq, Hkv, T, D = O.BF16, 2, 16, 4, 333, 128
    rng = np.random.default_rng(60 + bits + L)
    q = rand_bits(rng, (B, Hq, L, D), dtype)
    kx, vx = (rand_bits(rng, (B, Hkv, T, D), dtype) for _ in range(2))
    kq, ks, kb, _ = O.quantize(kx, dtype, 64, bits)
    vq, vs, vb, _ = O.quantize(vx, dtype, 64, bits)
    t = lambda a: torch.from_numpy(a.view(np.int32)).cuda()
    args = (dev(q, dtype), (t(kq), dev(ks, dtype), dev(kb, dtype)),
            (t(vq), dev(vs, dtype), dev(vb, dtype)), D ** -0.5)
    run = lambda: values(vkv.quantized_scaled_dot_product_attention(
        *args, mask=mask, group_size=64, bits=bits), dtype)
    got = run()
    f = lambda a: O.to_f32(a, dtype)
    ref, wb = qref(f(q), dtype, kq, f(ks), f(kb), vq, f(vs), f(vb), D ** -0.5, 64, bits,
                   mask=mask, rounding=O.REF_CHUNK)
    tol = qattn_tol(dtype, ref, wb)
    assert_within(got, ref, tol, "oracle", wb)
    monkeypatch.setattr(OPTIONS, "generic_attention", 1)
    assert_within(got, run(), attn_tol(dtype, ref) + 2 * wb, "generic", wb)
