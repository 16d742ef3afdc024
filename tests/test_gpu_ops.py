"""GPU parity of the stateless operators through the C ABI against the CPU
oracle: affine quantize / dequantize (bit-exact), float SDPA and quantized
SDPA (tolerance), on seeded inputs including the reference's own known
answers."""
import numpy as np
import pytest
import torch

import mlx_random as mr
import oracle as O
import vkv
from gpu_util import OPTIONS, assert_qclose, assert_within, qattn_tol, qref, attn_tol, dev, host, rand_bits, values

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype", [O.F16, O.BF16, O.F32])
@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("group", [32, 64, 128])
def test_quantize_bit_exact(dtype, bits, group):
    rng = np.random.default_rng(100 * bits + group + dtype)
    w = rand_bits(rng, (3, 5, 7, 256), dtype, outliers=4)
    # edge rows: zeros, constant, all negative, one huge value, tiny values
    w[0, 0, 0] = O.from_f32(np.zeros(256, np.float32), dtype)
    w[0, 0, 1] = O.from_f32(np.full(256, 3.25, np.float32), dtype)
    w[0, 0, 2] = O.from_f32(-np.abs(rng.standard_normal(256)).astype(np.float32) - 0.1, dtype)
    big = np.zeros(256, np.float32)
    big[17] = 1000.0
    w[0, 0, 3] = O.from_f32(big, dtype)
    w[0, 0, 4] = O.from_f32((rng.standard_normal(256) * 1e-6).astype(np.float32), dtype)
    wq, sc, bi = vkv.quantized(dev(w, dtype), group_size=group, bits=bits)
    torch.cuda.synchronize()
    rq, rs, rb, ties = O.quantize(w, dtype, group, bits)
    assert np.array_equal(host(wq), rq)
    assert np.array_equal(host(sc).view(rs.dtype), rs)
    assert np.array_equal(host(bi).view(rb.dtype), rb)


def test_quantize_strided_input_and_reference_aggregate(golden):
    """A non-contiguous view quantizes like its contiguous copy; the seed-869
    reference aggregate (IntegrationTests.swift:3890-3923) holds on the GPU."""
    g = golden["quantize_uniform_8bit"]
    w = mr.uniform(mr.KeySequence(g["seed"]), tuple(g["shape"]))
    wq, sc, bi = vkv.quantized(dev(w, O.F32), group_size=64, bits=8)
    wsum = int(host(wq).astype(np.uint64).sum()) % (1 << 32)
    assert np.float32(wsum) == np.float32(g["wq_sum"])
    assert abs(host(sc).astype(np.float64).sum() - g["scales_sum"]) < 1e-5 * abs(g["scales_sum"])
    rng = np.random.default_rng(3)
    base = dev(rand_bits(rng, (4, 6, 9, 128), O.BF16), O.BF16)
    view = base.transpose(1, 2)  # [4, 9, 6, 128], last dim contiguous
    a = vkv.quantized(view, 64, 4)
    b = vkv.quantized(view.contiguous(), 64, 4)
    for x, y in zip(a, b):
        assert torch.equal(x, y)


@pytest.mark.parametrize("dtype", [O.F16, O.BF16, O.F32])
@pytest.mark.parametrize("bits", [4, 8])
def test_dequantize_bit_exact(dtype, bits):
    rng = np.random.default_rng(7 + bits + dtype)
    w = rand_bits(rng, (16, 128), dtype, outliers=2)
    rq, rs, rb, _ = O.quantize(w, dtype, 64, bits)
    out = vkv.dequantized(torch.from_numpy(rq.view(np.int32)).cuda(), dev(rs, dtype),
                          dev(rb, dtype), 64, bits)
    ref = O.dequantize(rq, rs, rb, dtype, 64, bits)
    assert np.array_equal(host(out).view(ref.dtype), ref)


def test_sdpa_reference_known_answer(golden):
    """MLXFastKernelTests.swift:101-111 on the GPU."""
    g = golden["fast_sdpa_output"]
    s = mr.KeySequence(g["seed"])
    q, k, v = (mr.uniform(s, tuple(g[n])) for n in ("q_shape", "kv_shape", "kv_shape"))
    out = vkv.scaled_dot_product_attention(dev(q, O.F32), dev(k, O.F32), dev(v, O.F32), g["scale"])
    assert abs(float(out.double().sum()) - g["sum"]) <= g["accuracy"]


@pytest.mark.parametrize("dtype", [O.F16, O.BF16, O.F32])
@pytest.mark.parametrize("shape", [(1, 32, 8, 1, 513, 128), (2, 8, 2, 3, 77, 80),
                                   (1, 4, 4, 1, 4100, 64), (3, 16, 8, 1, 1, 256)])
def test_sdpa_matches_oracle(dtype, shape):
    B, Hq, Hkv, L, T, D = shape
    rng = np.random.default_rng(T + D + dtype)
    q, k, v = (rand_bits(rng, s, dtype) for s in ((B, Hq, L, D), (B, Hkv, T, D), (B, Hkv, T, D)))
    scale = D ** -0.5
    out = vkv.scaled_dot_product_attention(dev(q, dtype), dev(k, dtype), dev(v, dtype), scale)
    f = lambda a: O.to_f32(a, dtype) if dtype != O.F32 else a
    ref = O.sdpa(f(q), f(k), f(v), scale)
    got = values(out, dtype)
    assert (np.abs(got - ref) <= attn_tol(dtype, ref)).all()


@pytest.mark.parametrize("dtype", [O.BF16, O.F16, O.F32])
@pytest.mark.parametrize("Hq,Hkv,D", [(16, 8, 256), (32, 8, 128), (12, 4, 64), (12, 1, 128), (8, 8, 64)])
@pytest.mark.parametrize("mask", [None, "bool", "add"])
def test_sdpa_decode_one_token(dtype, Hq, Hkv, D, mask, monkeypatch):
    """One query token over dense K/V (the dense decode kernel): GQA 1 to 12
    (head groups of up to 8), K/V as strided views of a longer buffer (a
    cache's [.., cap, D] storage), lengths that end inside a 64-token step,
    per-head bool masks with an empty row, additive masks; against the oracle
    and against the generic kernel."""
    rng = np.random.default_rng(Hq * 7 + D + dtype + (0 if mask is None else len(mask)))
    B, T, cap = 3, 1000, 1100
    q = rand_bits(rng, (B, Hq, 1, D), dtype)
    kb = rand_bits(rng, (B, Hkv, cap, D), dtype)
    vb = rand_bits(rng, (B, Hkv, cap, D), dtype)
    k_dev, v_dev = dev(kb, dtype)[:, :, :T], dev(vb, dtype)[:, :, :T]
    k, v = kb[:, :, :T], vb[:, :, :T]
    if mask == "bool":
        m = rng.random((B, Hq, 1, T)) > 0.3
        m[1, 2, 0] = False  # fully masked row -> zeros
        m_dev, m_ref = torch.from_numpy(m).cuda(), m
    elif mask == "add":
        m = (rng.standard_normal((1, T)) * 2).astype(np.float32)
        m[0, :7] = -np.inf
        m_dev, m_ref = torch.from_numpy(m).cuda(), m
    else:
        m_dev = m_ref = None
    scale = D ** -0.5
    out = vkv.scaled_dot_product_attention(dev(q, dtype), k_dev, v_dev, scale, mask=m_dev)
    f = lambda a: O.to_f32(a, dtype) if dtype != O.F32 else a
    ref = O.sdpa(f(q), f(k), f(v), scale, mask=m_ref, q_dtype=dtype)
    got = values(out, dtype)
    assert (np.abs(got - ref) <= attn_tol(dtype, ref)).all()
    if mask == "bool":
        assert (got[1, 2, 0] == 0).all()
    monkeypatch.setattr(OPTIONS, "generic_attention", 1)
    gen = values(vkv.scaled_dot_product_attention(dev(q, dtype), k_dev, v_dev, scale, mask=m_dev),
                 dtype)
    assert (np.abs(got - gen) <= attn_tol(dtype, ref)).all()


@pytest.mark.parametrize("mask", ["causal", "bool", "add", "bool_empty_row"])
def test_sdpa_masks(mask):
    dtype = O.BF16
    rng = np.random.default_rng(11)
    B, Hq, Hkv, L, T, D = 2, 8, 4, 5, 37, 128
    q, k, v = (rand_bits(rng, s, dtype) for s in ((B, Hq, L, D), (B, Hkv, T, D), (B, Hkv, T, D)))
    if mask == "causal":
        m_dev, m_ref = "causal", "causal"
    elif mask.startswith("bool"):
        m = rng.random((B, 1, L, T)) > 0.4
        if mask == "bool_empty_row":
            m[1, 0, 2] = False  # fully masked row -> zeros
        m_dev, m_ref = torch.from_numpy(m).cuda(), m
    else:
        m = (rng.standard_normal((L, T)) * 3).astype(np.float32)
        m[0, :5] = -np.inf
        m_dev, m_ref = torch.from_numpy(m).cuda(), m
    out = vkv.scaled_dot_product_attention(dev(q, dtype), dev(k, dtype), dev(v, dtype), 0.1,
                                           mask=m_dev)
    f = lambda a: O.to_f32(a, dtype)
    ref = O.sdpa(f(q), f(k), f(v), 0.1, mask=m_ref, q_dtype=dtype)
    got = values(out, dtype)
    assert (np.abs(got - ref) <= attn_tol(dtype, ref)).all()
    if mask == "bool_empty_row":
        assert (got[1, :, 2] == 0).all()


@pytest.mark.parametrize("dtype", [O.F16, O.BF16])
@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("mask", [None, "causal", "bool"])
def test_quantized_sdpa_matches_oracle(dtype, bits, mask):
    rng = np.random.default_rng(bits * 3 + dtype)
    B, Hq, Hkv, L, T, D = 2, 32, 8, 1 if mask is None else 4, 300, 128
    q = rand_bits(rng, (B, Hq, L, D), dtype)
    kx, vx = (rand_bits(rng, (B, Hkv, T, D), dtype, outliers=4) for _ in range(2))
    kq, ks, kb, _ = O.quantize(kx, dtype, 64, bits)
    vq, vs, vb, _ = O.quantize(vx, dtype, 64, bits)
    m_dev = m_ref = None
    if mask == "causal":
        m_dev = m_ref = "causal"
    elif mask == "bool":
        m = rng.random((B, Hq, L, T)) > 0.5
        m[0, 3, 1] = False  # fully masked row -> mean of V (finfo.min fill)
        m_dev, m_ref = torch.from_numpy(m).cuda(), m
    t = lambda a: torch.from_numpy(a.view(np.int32)).cuda()
    scale = D ** -0.5
    out = vkv.quantized_scaled_dot_product_attention(
        dev(q, dtype), (t(kq), dev(ks, dtype), dev(kb, dtype)), (t(vq), dev(vs, dtype), dev(vb, dtype)),
        scale, mask=m_dev, group_size=64, bits=bits)
    f = lambda a: O.to_f32(a, dtype)
    ref, wb = qref(f(q), dtype, kq, f(ks), f(kb), vq, f(vs), f(vb), scale, 64, bits,
                   mask=m_ref)
    got = values(out, dtype)
    assert_qclose(got, ref, wb, dtype, f"{dtype} {bits} {mask}")


@pytest.mark.parametrize("path", ["decode", "generic", "prefill", "router"])
@pytest.mark.parametrize("dtype", [O.BF16, O.F16])
def test_sdpa_sinks(path, dtype, monkeypatch):
    """Attention sinks (MLXFast.scaledDotProductAttention(..., sinks:),
    sdpa_vector.h:93-96, :257-260) on every float path: the dense decode
    kernel (one token, a fully masked row keeps only its sink and yields
    zeros), the generic kernel, the multi-query prefill kernel (causal), and
    the router over a KVCacheSimple; against the oracle."""
    rng = np.random.default_rng(60 + dtype + len(path))
    B, Hq, Hkv, D = 2, 16, 4, 128
    L, T = (1, 700) if path in ("decode", "generic") else (40, 40)
    q = rand_bits(rng, (B, Hq, L, D), dtype)
    k = rand_bits(rng, (B, Hkv, T, D), dtype)
    v = rand_bits(rng, (B, Hkv, T, D), dtype)
    sk = O.from_f32((rng.standard_normal(Hq) * 2 + 5).astype(np.float32), dtype)
    f = lambda a: O.to_f32(a, dtype)
    scale = D ** -0.5
    if L == 1:
        m = rng.random((B, Hq, 1, T)) > 0.3
        m[1, 3, 0] = False
        m_dev, m_ref = torch.from_numpy(m).cuda(), m
    else:
        m_dev = m_ref = "causal"
    if path == "generic":
        monkeypatch.setattr(OPTIONS, "generic_attention", 1)
    if path == "router":
        c = vkv.KVCacheSimple()
        out = vkv.attention_with_cache_update(dev(q, dtype), dev(k, dtype), dev(v, dtype), c, scale,
                                              mask=m_dev, sinks=dev(sk, dtype))
        assert c.offset == T
    else:
        out = vkv.scaled_dot_product_attention(dev(q, dtype), dev(k, dtype), dev(v, dtype), scale,
                                               mask=m_dev, sinks=dev(sk, dtype))
    ref = O.sdpa(f(q), f(k), f(v), scale, mask=m_ref, q_dtype=dtype, sinks=f(sk))
    got = values(out, dtype)
    assert_within(got, ref, attn_tol(dtype, ref), path)
    if L == 1:
        assert (got[1, 3, 0] == 0).all()
    # the sinks change the result (they are not ignored)
    plain = O.sdpa(f(q), f(k), f(v), scale, mask=m_ref, q_dtype=dtype)
    assert np.abs(plain - ref).max() > 0.1 * np.abs(plain).max()


def test_quantized_cache_refuses_sinks():
    c = vkv.QuantizedKVCache(64, 4)
    x = torch.zeros((1, 2, 1, 64), dtype=torch.bfloat16, device="cuda")
    q = torch.zeros((1, 4, 1, 64), dtype=torch.bfloat16, device="cuda")
    with pytest.raises(vkv.VKVError, match="sinks"):
        vkv.attention_with_cache_update(q, x, x, c, 0.125,
                                        sinks=torch.zeros(4, dtype=torch.bfloat16, device="cuda"))
    assert c.offset == 0


@pytest.mark.parametrize("generic", [False, True])
def test_sdpa_additive_mask_in_query_dtype(generic, monkeypatch):
    """Additive masks are read in the query dtype (sdpa_vector.h:15-38,
    :105-121): with f16 queries an f32 mask of -1e9 rounds to -inf and
    empties the row (zeros); with bf16 queries a bf16 mask of -1e9 stays
    finite, the fp32 scores collapse to -1e9 and the row averages V."""
    if generic:
        monkeypatch.setattr(OPTIONS, "generic_attention", 1)
    rng = np.random.default_rng(70)
    B, Hq, Hkv, T, D = 1, 4, 2, 300, 64
    for dtype, mdt in ((O.F16, np.float32), (O.BF16, None)):
        q = rand_bits(rng, (B, Hq, 1, D), dtype)
        k = rand_bits(rng, (B, Hkv, T, D), dtype)
        v = rand_bits(rng, (B, Hkv, T, D), dtype)
        m = (rng.standard_normal((B, Hq, 1, T)) * 2).astype(np.float32)
        m[0, 1] = -1e9
        if mdt is None:
            mb = O.from_f32(m, dtype)
            m_dev, m_ref = dev(mb, dtype), O.to_f32(mb, dtype)
        else:
            m_dev, m_ref = torch.from_numpy(m).cuda(), m
        f = lambda a: O.to_f32(a, dtype)
        out = values(vkv.scaled_dot_product_attention(dev(q, dtype), dev(k, dtype), dev(v, dtype),
                                                      0.125, mask=m_dev), dtype)
        ref = O.sdpa(f(q), f(k), f(v), 0.125, mask=m_ref, q_dtype=dtype)
        assert_within(out, ref, attn_tol(dtype, ref), f"dtype {dtype}")
        if dtype == O.F16:
            assert (out[0, 1] == 0).all()
        else:
            mean_v = f(v)[0, 0].mean(0)  # head 1 reads kv head 0
            assert np.abs(out[0, 1, 0] - mean_v).max() < 2e-2
