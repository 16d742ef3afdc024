"""A seeded sweep of the paged matrix-core decode over affine blocks (the
config-3 path: quantizedScaledDotProductAttention, KVCache.swift:1909-1997,
over per-sequence lengths in a block pool) against the oracle's quantized
SDPA over the same codes: random sequence counts (1-40, an empty and a
one-token sequence among them when there are three or more), lengths up to
5000, kv heads 1-8, query heads a kv head 1-12 (two head groups past 8),
head dims 64 / 128 / 256, 4 / 8 bits, groups of 64 or 128, bf16 / f16, ×20
outlier channels.  The bar is the fp32-softmax contract (2e-2 + 1 ulp + the
reference's weight-rounding term); the kernel timing counts show the
matrix-core kernel ran."""
import numpy as np
import pytest
import torch

import oracle as O
import vkv
from gpu_util import assert_qclose, dev, qref, rand_bits, values
from test_gpu_decode_g128 import decode, scene

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("seed", range(10))
def test_paged_decode_sweep(seed):
    rng = np.random.default_rng(9900 + seed)
    dtype = O.BF16 if seed % 2 == 0 else O.F16
    D = int(rng.choice([64, 128, 256]))
    bits = int(rng.choice([4, 8]))
    group = 128 if D >= 128 and rng.random() < 0.3 else 64
    Hkv = int(rng.integers(1, 9))
    rep = int(rng.choice([1, 2, 3, 4, 5, 8, 12]))
    n = int(rng.integers(1, 41))
    # bounded so the oracle finishes within seconds
    lens = [int(x) for x in rng.integers(1, 5001, n)]
    while sum(lens) * Hkv * rep * D > 4e8:
        lens = [max(1, L // 2) for L in lens]
    if n >= 3:
        lens[1], lens[2] = 0, 1
    print(f"paged decode sweep {seed}: dtype {dtype} bits {bits} group {group} D {D} Hkv {Hkv} "
          f"rep {rep} n {n} max len {max(lens)}", flush=True)
    pool, view, keys, vals, keep = scene(rng, bits, group, lens, Hkv, D, dtype)
    q = rand_bits(rng, (n, Hkv * rep, D), dtype)
    out, n_dec = decode(dev(q, dtype), view, D, timed=True)
    assert n_dec >= 1, "the matrix-core decode did not run"
    got = values(out, dtype)
    f = lambda a: O.to_f32(a, dtype)
    for s, L in enumerate(lens):
        if L == 0:
            assert not got[s].any(), "an empty sequence yields zeros"
            continue
        rk = O.quantize(np.ascontiguousarray(keys[s][:L].transpose(1, 0, 2)), dtype, group, bits)
        rv = O.quantize(np.ascontiguousarray(vals[s][:L].transpose(1, 0, 2)), dtype, group, bits)
        ref, wb = (x[0, :, 0] for x in qref(f(q[s])[None, :, None], dtype, rk[0][None],
                                            f(rk[1])[None], f(rk[2])[None], rv[0][None],
                                            f(rv[1])[None], f(rv[2])[None], D ** -0.5, group,
                                            bits))
        assert_qclose(got[s], ref, wb, dtype, f"case {seed} seq {s} (len {L})")
