"""Which kernel takes a one-token decode over f32 rows (MLXFast
scaledDotProductAttention, sdpa_vector.h:15-177): the float decode kernel
where a wave's registers hold the step, the generic kernel for f32 rows at
128 dims with more than 4 query heads a kv head and at 256 dims with more
than 2 (those variants spilled to scratch and ran 1.9-4.7x slower).  The
kernel timing counts show the route; both routes are within the f32 bar
(1e-4 + 1 ulp) of the oracle's float SDPA."""
import numpy as np
import pytest
import torch

import oracle as O
import vkv
from gpu_util import assert_within, attn_tol, dev, rand_bits, values

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("D,rep,fdecode", [(64, 8, True), (128, 4, True), (128, 8, False),
                                           (256, 2, True), (256, 4, False), (256, 8, False)])
def test_f32_decode_route(D, rep, fdecode):
    rng = np.random.default_rng(9300 + D + rep)
    B, Hkv, T, dtype = 2, 2, 700, O.F32
    print(f"f32 decode route: D {D} rep {rep}", flush=True)
    k = rand_bits(rng, (B, Hkv, T, D), dtype)
    v = rand_bits(rng, (B, Hkv, T, D), dtype)
    q = rand_bits(rng, (B, Hkv * rep, 1, D), dtype)
    vkv.kernel_timing(True)
    out = vkv.scaled_dot_product_attention(dev(q, dtype), dev(k, dtype), dev(v, dtype), D ** -0.5)
    torch.cuda.synchronize()
    _, n = vkv.kernel_timing_read(vkv.TIME_FDECODE)
    vkv.kernel_timing(False)
    assert (n > 0) == fdecode, f"float decode launches: {n}"
    ref = O.sdpa(q, k, v, D ** -0.5)
    assert_within(values(out, dtype), ref, attn_tol(dtype, ref), f"D {D} rep {rep}")
