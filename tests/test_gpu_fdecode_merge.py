"""The float decode's split merge (sdpa_vector_2pass_2, sdpa_vector.h:
320-394) on both of its paths: inside the decode launch (the part that
counts in last merges through device-coherent loads and zeroes its counter
again) where the merge is small, and in attn_combine_kernel otherwise.
Each path is checked against the oracle's float SDPA over several calls in
a row (the counters must be back at zero after every launch) and under HIP
graph replay (the counters reset inside the graph, no memset recorded)."""
import numpy as np
import pytest
import torch

import oracle as O
import vkv
from gpu_util import assert_within, attn_tol, dev, rand_bits, values

pytestmark = pytest.mark.gpu

# (B, Hkv, Hq, T, D, dtype): 18 parts x 128 dims x 4 heads merges inside;
# 32 parts x 256 dims x 2 heads in the merge launch; one head per group
# (rep 1) and 8 heads per group (rep 8) inside
SHAPES = [(2, 4, 16, 576, 128, O.BF16), (4, 8, 16, 1024, 256, O.BF16),
          (1, 8, 8, 700, 64, O.F16), (2, 2, 16, 300, 128, O.F32)]


def _ref(q, k, v, dtype, scale):
    f = (lambda a: O.to_f32(a, dtype)) if dtype != O.F32 else (lambda a: a)
    return O.sdpa(f(q), f(k), f(v), scale)


@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "x".join(map(str, s[:5])))
def test_decode_calls_in_a_row(shape):
    B, Hkv, Hq, T, D, dtype = shape
    rng = np.random.default_rng(1500 + T + D)
    k = rand_bits(rng, (B, Hkv, T, D), dtype)
    v = rand_bits(rng, (B, Hkv, T, D), dtype)
    kd, vd = dev(k, dtype), dev(v, dtype)
    print(f"fdecode merge: shape {shape}", flush=True)
    for call in range(4):
        q = rand_bits(rng, (B, Hq, 1, D), dtype)
        out = vkv.scaled_dot_product_attention(dev(q, dtype), kd, vd, D ** -0.5)
        torch.cuda.synchronize()
        ref = _ref(q, k, v, dtype, D ** -0.5)
        assert_within(values(out, dtype), ref, attn_tol(dtype, ref), f"call {call}")


@pytest.mark.parametrize("shape", SHAPES[:2], ids=["merge_inside", "merge_launch"])
def test_decode_under_graph_replay(shape):
    B, Hkv, Hq, T, D, dtype = shape
    rng = np.random.default_rng(1600 + D)
    k = rand_bits(rng, (B, Hkv, T, D), dtype)
    v = rand_bits(rng, (B, Hkv, T, D), dtype)
    kd, vd = dev(k, dtype), dev(v, dtype)
    qin = torch.zeros((B, Hq, 1, D), dtype=torch.bfloat16, device="cuda")
    out = torch.empty_like(qin)
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):  # workspace and counters exist before the capture
        vkv.scaled_dot_product_attention(qin, kd, vd, D ** -0.5, out=torch.empty_like(out))
    torch.cuda.synchronize()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            vkv.scaled_dot_product_attention(qin, kd, vd, D ** -0.5, out=out)
    torch.cuda.synchronize()
    for r in range(4):
        q = rand_bits(rng, (B, Hq, 1, D), dtype)
        qin.copy_(dev(q, dtype))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        ref = _ref(q, k, v, dtype, D ** -0.5)
        assert_within(values(out, dtype), ref, attn_tol(dtype, ref), f"replay {r}")
        # eager calls between the replays use the same counters
        eager = vkv.scaled_dot_product_attention(qin, kd, vd, D ** -0.5)
        torch.cuda.synchronize()
        assert torch.equal(eager, out)
