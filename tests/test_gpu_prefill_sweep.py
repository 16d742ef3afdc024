"""A seeded sweep of multi-query attention over dense bf16 / f16 K/V (the
matrix-core chunk path of vkv_sdpa, MLXFast scaledDotProductAttention with
L >= 2 query tokens, sdpa_vector.h / steel attention semantics) against the
oracle's float SDPA: random batch rows (1-3), kv heads (1, 2, 4, 8), query
heads a kv head (1, 2, 3, 4, 6, 8), head dims 64 / 128 / 256, query counts
2-600 and key counts from the query count up to 3000 (not multiples of the
32-token tile or the 256-row block), no mask or the causal mask of the
chunk's offset, and a third of the cases over strided slices of larger
cache buffers.  The bar is the float attention bar: 2e-2 + 1 ulp."""
import numpy as np
import pytest
import torch

import oracle as O
import vkv
from gpu_util import assert_within, attn_tol, dev, rand_bits, values

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("seed", range(10))
def test_prefill_sweep(seed):
    rng = np.random.default_rng(9700 + seed)
    dtype = O.BF16 if seed % 2 == 0 else O.F16
    D = int(rng.choice([64, 128, 256]))
    Hkv = int(rng.choice([1, 2, 4, 8]))
    rep = int(rng.choice([1, 2, 3, 4, 6, 8]))
    B = int(rng.integers(1, 4))
    # bounded so the oracle's float64 SDPA stays within seconds
    L = int(rng.integers(2, 601))
    T = int(rng.integers(L, 3001))
    while B * Hkv * rep * L * T * D > 1.5e9:
        L = max(2, L // 2)
        T = max(L, T // 2)
    mask = "causal" if rng.random() < 0.6 else None
    strided = rng.random() < 0.33
    print(f"prefill sweep {seed}: dtype {dtype} B {B} Hkv {Hkv} rep {rep} L {L} T {T} D {D} "
          f"mask {mask} strided {strided}", flush=True)
    q = rand_bits(rng, (B, Hkv * rep, L, D), dtype)
    k = rand_bits(rng, (B, Hkv, T, D), dtype)
    v = rand_bits(rng, (B, Hkv, T, D), dtype)
    if strided:  # slices of cache-like buffers: head stride cap * D
        cap = T + int(rng.integers(1, 300))
        kb = torch.zeros((B, Hkv, cap, D), dtype=dev(k, dtype).dtype, device="cuda")
        vb = torch.zeros_like(kb)
        kb[:, :, :T] = dev(k, dtype)
        vb[:, :, :T] = dev(v, dtype)
        kd, vd = kb[:, :, :T], vb[:, :, :T]
    else:
        kd, vd = dev(k, dtype), dev(v, dtype)
    out = vkv.scaled_dot_product_attention(dev(q, dtype), kd, vd, D ** -0.5, mask=mask)
    torch.cuda.synchronize()
    f = lambda a: O.to_f32(a, dtype)
    ref = O.sdpa(f(q), f(k), f(v), D ** -0.5, mask=mask)
    assert_within(values(out, dtype), ref, attn_tol(dtype, ref), f"case {seed}")
