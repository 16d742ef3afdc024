"""QuantizedKVCache at the Llama-3-8B layer shape of the quantized-cache
workload: batch 8, 8 kv heads x 128 dims, 32 query heads, a 4096-token
context, bf16 K/V ~ N(0,1) with 4 random channels per head scaled x20,
affine g64 at 4 and 8 bits.

The cache is filled by one prefill update and one decode update
(QuantizedKVCache.updateQuantized, KVCache.swift:1049-1122), its state is
checked bit-exact against the restatement, and the decode step's attention
(quantizedScaledDotProductAttention, KVCache.swift:1909-1997, through the
attention router) is checked against the oracle with the reference's
rounding: scores and softmax weights stored in bf16.  On this data that
rounding moves outputs by up to ~1 against exact arithmetic, so the check
is only meaningful against the rounded oracle; the test also asserts that
the exact-arithmetic oracle is NOT within the tolerance, i.e. that the data
really exercises the rounding."""
import numpy as np
import pytest

import kvcache_ref as R
import oracle as O
import vkv
from gpu_util import OPTIONS, assert_within, attn_tol, dev, host, values

pytestmark = pytest.mark.gpu


def outlier_kv(rng, shape, dtype, n_out=4, factor=20.0):
    """N(0,1) with n_out random channels per (batch, head) scaled by factor."""
    x = rng.standard_normal(shape).astype(np.float32)
    B, H = shape[0], shape[1]
    for b in range(B):
        for h in range(H):
            x[b, h, :, rng.choice(shape[-1], n_out, replace=False)] *= factor
    return O.from_f32(x, dtype)


@pytest.mark.parametrize("ref_mode", [1, 0], ids=["reference_softmax", "fp32_softmax"])
@pytest.mark.parametrize("bits", [4, 8])
def test_config2_decode_step_reference_rounding(bits, ref_mode, monkeypatch):
    """With the reference softmax (the reference_softmax option) the bar is
    2e-2 + 1 ulp + the score-boundary term alone; with the fp32 softmax of
    the single-pass kernel it adds the weight term the reference's bf16
    weights put on this data (the documented contract of that mode)."""
    dtype, B, Hkv, Hq, D, T = O.BF16, 8, 8, 32, 128, 4096
    monkeypatch.setattr(OPTIONS, "reference_softmax", ref_mode)
    rng = np.random.default_rng(200 + bits)
    print(f"config 2: bits {bits} ref {ref_mode} B {B} Hkv {Hkv} Hq {Hq} D {D} T {T}", flush=True)
    c = vkv.QuantizedKVCache(group_size=64, bits=bits)
    r = R.QuantizedKVCacheRef(64, bits)
    k0, v0 = (outlier_kv(rng, (B, Hkv, T - 1, D), dtype) for _ in range(2))
    c.update_quantized(dev(k0, dtype), dev(v0, dtype))
    r.update_quantized(k0, v0, dtype)
    k1, v1 = (outlier_kv(rng, (B, Hkv, 1, D), dtype) for _ in range(2))
    q = O.from_f32(rng.standard_normal((B, Hq, 1, D)).astype(np.float32), dtype)
    out = vkv.attention_with_cache_update(dev(q, dtype), dev(k1, dtype), dev(v1, dtype), c,
                                          D ** -0.5)
    r.update_quantized(k1, v1, dtype)
    assert c.offset == r.offset == T and c.meta_state == r.meta_state
    for got, want in zip(c.state, r.state):
        assert np.array_equal(host(got), want)
    got = values(out, dtype)
    kq, ks, kb, vq, vs, vb = r.state
    f = lambda a: O.to_f32(a, dtype)
    args = (f(q), dtype, kq, f(ks), f(kb), vq, f(vs), f(vb), D ** -0.5, 64, bits)
    ref, wb, fb = O.quantized_sdpa(*args, rounding=O.REF_DECODE, bound=True, flip=True)
    err = np.abs(got - ref)
    bound = fb if ref_mode else wb
    tol = attn_tol(dtype, ref) + bound
    print(f"  max |got - ref| {err.max():.4f}, max bound {bound.max():.4f} "
          f"(score-boundary term {fb.max():.4f}), "
          f"max excess over 2e-2 + 1 ulp {(err - attn_tol(dtype, ref)).max():.4f}", flush=True)
    assert_within(got, ref, tol, f"bits {bits}", bound)
    exact = O.quantized_sdpa(*args, rounding=O.EXACT)
    assert not (np.abs(got - exact) <= attn_tol(dtype, exact)).all()
