"""A seeded sweep of one-token decode attention over dense float K/V (the
float decode kernel of vkv_sdpa, MLXFast scaledDotProductAttention with one
query token, sdpa_vector.h:15-177 and its split form :179-394) against the
oracle's float SDPA: random batch rows (1-4), kv heads (1-8), query heads a
kv head (1-8, odd ones included), head dims 64 / 128 / 256, bf16 / f16 / f32,
token counts 1-5000 (not multiples of the 32-token step), so the launch
takes the workgroup form, the split form merging inside the launch or the
merge launch by its size; no mask, a bool mask or an additive mask in the
query dtype, with or without sinks; a third of the cases over strided
slices of larger cache buffers.  Bar: 2e-2 (1e-4 for f32) + 1 ulp."""
import numpy as np
import pytest
import torch

import oracle as O
import vkv
from gpu_util import assert_within, attn_tol, dev, rand_bits, values

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("seed", range(12))
def test_fdecode_sweep(seed):
    rng = np.random.default_rng(9800 + seed)
    dtype = (O.BF16, O.F16, O.F32)[seed % 3]
    D = int(rng.choice([64, 128, 256]))
    Hkv = int(rng.integers(1, 9))
    rep = int(rng.integers(1, 9))
    B = int(rng.integers(1, 5))
    T = int(rng.choice([int(rng.integers(1, 64)), int(rng.integers(64, 1200)),
                        int(rng.integers(1200, 5001))]))
    mask_kind = rng.choice(["none", "bool", "add"])
    sinks = rng.random() < 0.3
    strided = rng.random() < 0.33
    Hq = Hkv * rep
    print(f"fdecode sweep {seed}: dtype {dtype} B {B} Hkv {Hkv} rep {rep} T {T} D {D} "
          f"mask {mask_kind} sinks {sinks} strided {strided}", flush=True)
    q = rand_bits(rng, (B, Hq, 1, D), dtype)
    k = rand_bits(rng, (B, Hkv, T, D), dtype)
    v = rand_bits(rng, (B, Hkv, T, D), dtype)
    f = (lambda a: O.to_f32(a, dtype)) if dtype != O.F32 else (lambda a: a)
    if strided:  # slices of cache-like buffers: head stride cap * D
        cap = T + int(rng.integers(1, 200))
        kb = torch.zeros((B, Hkv, cap, D), dtype=dev(k, dtype).dtype, device="cuda")
        vb = torch.zeros_like(kb)
        kb[:, :, :T] = dev(k, dtype)
        vb[:, :, :T] = dev(v, dtype)
        kd, vd = kb[:, :, :T], vb[:, :, :T]
    else:
        kd, vd = dev(k, dtype), dev(v, dtype)
    m_dev = m_ref = None
    if mask_kind == "bool":
        m = rng.random((B, Hq, 1, T)) > 0.3
        m[..., 0] = True  # no row left empty without a sink
        m_dev, m_ref = torch.from_numpy(m).cuda(), m
    elif mask_kind == "add":
        m = (rng.standard_normal((B, Hq, 1, T)) * 2).astype(np.float32)
        mb = O.from_f32(m, dtype) if dtype != O.F32 else m
        m_dev, m_ref = dev(mb, dtype), f(mb)
    sk = sk_dev = None
    if sinks:
        sk = (rng.standard_normal(Hq) * 2).astype(np.float32)
        sk = O.from_f32(sk, dtype) if dtype != O.F32 else sk
        sk_dev = dev(sk, dtype)
    out = vkv.scaled_dot_product_attention(dev(q, dtype), kd, vd, D ** -0.5, mask=m_dev,
                                           sinks=sk_dev)
    torch.cuda.synchronize()
    ref = O.sdpa(f(q), f(k), f(v), D ** -0.5, mask=m_ref, q_dtype=dtype,
                 sinks=None if sk is None else f(sk))
    assert_within(values(out, dtype), ref, attn_tol(dtype, ref), f"case {seed}")
