"""Decode calls on two streams at once.  Each (device, stream) keeps its own
split-K workspace and in-launch merge counters, so launches that overlap on
two streams give the bits each gives alone: the paged matrix-core decode
over affine blocks (vkv_paged_sdpa, its partials merged inside the launch)
and the float decode (vkv_sdpa with one query token, merging small splits
inside its launch), six calls a stream with no synchronization between
them."""
import numpy as np
import pytest
import torch

import oracle as O
import vkv
from gpu_util import dev, host, rand_bits
from test_zz_no_alloc import scene

pytestmark = pytest.mark.gpu


def _two_streams(call_a, call_b, outs_a, outs_b):
    """call_a(out, stream) / call_b(out, stream) into each preallocated
    output, alternating between two new streams, then one synchronize."""
    cur = torch.cuda.current_stream()
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    s1.wait_stream(cur)
    s2.wait_stream(cur)
    for oa, ob in zip(outs_a, outs_b):
        with torch.cuda.stream(s1):
            call_a(oa, s1)
        with torch.cuda.stream(s2):
            call_b(ob, s2)
    torch.cuda.synchronize()


def test_paged_decode_on_two_streams():
    rng = np.random.default_rng(9100)
    dtype, bits, Hkv, D, rep = O.BF16, 4, 8, 128, 4
    pa = scene(rng, bits, [int(x) for x in rng.integers(1, 1500, 24)], Hkv, D)
    pb = scene(rng, bits, [int(x) for x in rng.integers(1, 3000, 17)], Hkv, D)
    qa = dev(rand_bits(rng, (24, Hkv * rep, D), dtype), dtype)
    qb = dev(rand_bits(rng, (17, Hkv * rep, D), dtype), dtype)
    print("paged decode on two streams", flush=True)
    want_a = vkv.paged_attention(qa, pa[1], D ** -0.5)
    want_b = vkv.paged_attention(qb, pb[1], D ** -0.5)
    outs_a = [torch.empty_like(want_a) for _ in range(6)]
    outs_b = [torch.empty_like(want_b) for _ in range(6)]
    torch.cuda.synchronize()
    _two_streams(lambda o, s: vkv.paged_attention(qa, pa[1], D ** -0.5, stream=s, out=o),
                 lambda o, s: vkv.paged_attention(qb, pb[1], D ** -0.5, stream=s, out=o),
                 outs_a, outs_b)
    for i, (oa, ob) in enumerate(zip(outs_a, outs_b)):
        assert np.array_equal(host(oa), host(want_a)), f"stream 1 call {i}"
        assert np.array_equal(host(ob), host(want_b)), f"stream 2 call {i}"


def test_float_decode_on_two_streams():
    rng = np.random.default_rng(9200)
    dtype = O.BF16
    # (B, Hkv, Hq, T, D): splits merged inside the launch, and a larger call
    # whose splits go to the merge launch
    shapes = [(2, 2, 16, 576, 128), (4, 8, 16, 1024, 256)]
    print("float decode on two streams", flush=True)
    calls, wants = [], []
    for B, Hkv, Hq, T, D in shapes:
        k = dev(rand_bits(rng, (B, Hkv, T, D), dtype), dtype)
        v = dev(rand_bits(rng, (B, Hkv, T, D), dtype), dtype)
        q = dev(rand_bits(rng, (B, Hq, 1, D), dtype), dtype)
        calls.append((q, k, v, D ** -0.5))
        wants.append(vkv.scaled_dot_product_attention(q, k, v, D ** -0.5))
    outs = [[torch.empty_like(w) for _ in range(6)] for w in wants]
    torch.cuda.synchronize()

    def run(c):
        q, k, v, sc = c
        return lambda o, s: vkv.scaled_dot_product_attention(q, k, v, sc, stream=s, out=o)

    _two_streams(run(calls[0]), run(calls[1]), outs[0], outs[1])
    for j in range(2):
        for i, o in enumerate(outs[j]):
            assert np.array_equal(host(o), host(wants[j])), f"shape {shapes[j]} call {i}"
