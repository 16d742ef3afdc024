"""Seeded sweeps that hold the decode's launch-level shortcuts to the plain
paths they replace, bit for bit (the same arithmetic, so any difference is
a lost, stale or raced partial or token):

* the paged matrix-core decode merging its split partials inside the launch
  (vkv_paged_sdpa: coherent partial stores, per-pair counters, the last wave
  of a pair merges) against vkv_paged_sdpa_noalloc, whose partials merge in
  qdecode_combine_kernel (sdpa_vector.h:320-394), over random batches:
  sequence counts, mixed lengths (empty and one-token sequences among
  them), 4 / 8 bits, 64 / 128 dims, bf16 / f16, 1 to 8 query heads a kv
  head, several calls in a row on one stream;
* the router's one-launch step over a QuantizedKVCache (the decode kernel
  writes the token, vkv_attention_with_cache_update) against the
  separate_token_write option's two launches, over random shapes and
  step counts, outputs and cache state."""
import numpy as np
import pytest
import torch

import oracle as O
import vkv
from gpu_util import OPTIONS, dev, host, rand_bits
from test_zz_no_alloc import scene

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("seed,bits,D,dtype", [(0, 4, 128, O.BF16), (1, 8, 128, O.BF16),
                                               (2, 4, 64, O.F16), (3, 8, 64, O.BF16),
                                               (4, 4, 128, O.F16), (5, 8, 128, O.F16)])
def test_in_launch_merge_equals_merge_launch(seed, bits, D, dtype):
    rng = np.random.default_rng(5000 + seed)
    Hkv = int(rng.choice([1, 2, 4]))
    rep = int(rng.choice([1, 2, 3, 4, 5, 8]))
    # many (sequence, kv head) pairs of short to medium lengths, so that the
    # launch averages at most 4 partials a pair (the in-launch merge) and
    # the no-allocation scratch holds its partials
    n = int(rng.integers(1, 400 // Hkv))
    lens = [int(x) for x in rng.integers(1, 800, n)]
    lens[0] = 1
    if n > 2:
        lens[1] = 0  # an empty sequence owns no block: zeros
    print(f"in-launch merge sweep {seed}: bits {bits} D {D} dtype {dtype} Hkv {Hkv} "
          f"rep {rep} n {n}", flush=True)
    pool, view, keys, vals, keep = scene(rng, bits, [max(L, 1) for L in lens], Hkv, D,
                                         dtype=dtype)
    keep[1].copy_(torch.tensor(lens, dtype=torch.int32))  # the real lengths, 0 included
    for call in range(3):  # calls in a row: the counters must be back at zero
        q = dev(rand_bits(rng, (n, Hkv * rep, D), dtype), dtype)
        want = vkv.paged_attention(q, view, D ** -0.5, out=torch.empty_like(q), noalloc=True)
        got = vkv.paged_attention(q, view, D ** -0.5)
        torch.cuda.synchronize()
        assert np.array_equal(host(got), host(want)), f"call {call}"
        if n > 2:
            assert not host(got)[1].any(), "an empty sequence yields zeros"


@pytest.mark.parametrize("seed,bits,D,dtype", [(0, 4, 128, O.BF16), (1, 8, 64, O.F16),
                                               (2, 4, 256, O.BF16), (3, 8, 128, O.F16)])
def test_one_launch_step_sweep(seed, bits, D, dtype, monkeypatch):
    rng = np.random.default_rng(6000 + seed)
    Hkv = int(rng.choice([1, 2, 4]))
    rep = int(rng.choice([1, 2, 4, 8]))
    B = int(rng.integers(1, 12))
    pre = int(rng.integers(2, 600))
    print(f"one-launch sweep {seed}: bits {bits} D {D} dtype {dtype} B {B} Hkv {Hkv} "
          f"rep {rep} prefill {pre}", flush=True)
    one, two = vkv.QuantizedKVCache(64, bits), vkv.QuantizedKVCache(64, bits)

    def rows(L):
        return (dev(rand_bits(rng, (B, Hkv * rep, L, D), dtype), dtype),
                dev(rand_bits(rng, (B, Hkv, L, D), dtype, outliers=2), dtype),
                dev(rand_bits(rng, (B, Hkv, L, D), dtype, outliers=2), dtype))

    q, k, v = rows(pre)
    for c in (one, two):
        vkv.attention_with_cache_update(q, k, v, c, D ** -0.5, mask="causal")
    for i in range(int(rng.integers(3, 12))):
        q, k, v = rows(1)
        monkeypatch.setattr(OPTIONS, "separate_token_write", 0)
        got = vkv.attention_with_cache_update(q, k, v, one, D ** -0.5)
        monkeypatch.setattr(OPTIONS, "separate_token_write", 1)
        want = vkv.attention_with_cache_update(q, k, v, two, D ** -0.5)
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"step {i}"
        if rng.random() < 0.2:
            t = int(rng.integers(1, 4))
            one.trim(t)
            two.trim(t)
    for i, (x, y) in enumerate(zip(one.state, two.state)):
        assert np.array_equal(host(x), host(y)), f"state array {i}"
