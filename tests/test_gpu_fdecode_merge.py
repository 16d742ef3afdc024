"""The float decode's split merge (sdpa_vector_2pass_2, sdpa_vector.h:
320-394) on its three paths: in LDS where one workgroup owns a whole (row,
kv head, head group) (small bf16 / f16 launches), inside the decode launch
(the part that counts in last merges through device-coherent loads and
zeroes its counter again) where the merge is small, and in
attn_combine_kernel otherwise.  Each path is checked against the oracle's
float SDPA over several calls in a row (the counters must be back at zero
after every launch) and under HIP graph replay (the counters reset inside
the graph, no memset recorded)."""
import numpy as np
import pytest
import torch

import oracle as O
import vkv
from gpu_util import assert_within, attn_tol, dev, rand_bits, values

pytestmark = pytest.mark.gpu

# (B, Hkv, Hq, T, D, dtype): 8 waves of a workgroup (one query head each
# at this size) merging in LDS; 32 parts x 256 dims x 2 heads in the merge
# launch; 8 heads per group (no workgroup form at 128 dims) merging inside
# the launch; the workgroup form at 64 dims, with parts fewer than waves;
# f32 merging inside the launch; the workgroup form of larger launches,
# which keeps the 8 / 4 heads of a kv head together
SHAPES = [(2, 4, 16, 576, 128, O.BF16), (4, 8, 16, 1024, 256, O.BF16),
          (2, 2, 16, 576, 128, O.BF16), (1, 8, 8, 100, 64, O.F16),
          (2, 2, 8, 300, 128, O.F32), (24, 4, 32, 64, 64, O.BF16),
          (40, 4, 16, 96, 128, O.F16)]


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


@pytest.mark.parametrize("shape", SHAPES[:3], ids=["workgroup", "merge_launch", "merge_inside"])
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
