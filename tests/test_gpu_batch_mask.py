"""createBatchCausalMask on the device (vkv_batch_causal_mask,
BatchEngine/BatchMask.swift:44-115): bit-exact with the restatement on the
reference's own cases, on random batches with windows and wrapped slots,
on a batch of 300 slots (two launches of the per-slot argument block) and
on sizes whose byte count is not a multiple of 16; and a batched
multi-token step -- per-slot keys zero-padded to the longest slot, as
BatchKVCache.padAndConcatenate pads them (BatchKVCache.swift:177-193) --
attended through the mask equals each slot's attention over its own keys."""
import numpy as np
import pytest
import torch

import kvcache_ref as R
import oracle as O
import vkv
from gpu_util import attn_tol, dev, rand_bits, values

pytestmark = pytest.mark.gpu


def _check(n, offsets, key_lens=None, window=None):
    got = vkv.batch_causal_mask(n, offsets, key_lens, window).cpu().numpy()
    want = R.batch_causal_mask(n, offsets, key_lens, window)
    assert got.shape == want.shape and np.array_equal(got, want), (n, offsets[:4], window)


def test_reference_cases():
    _check(1, [5, 3])
    _check(1, [5, 3], window=3)
    _check(1, [4, 4])
    _check(3, [2])
    _check(1, [100, 5], key_lens=[16, 6])
    _check(1, [40, 5], key_lens=[16, 6], window=16)


@pytest.mark.parametrize("seed", range(5))
def test_random_batches(seed):
    rng = np.random.default_rng(100 + seed)
    B = [3, 17, 300, 241, 1][seed]
    n = [1, 7, 3, 5, 13][seed]
    offsets = [int(x) for x in rng.integers(0, 700, B)]
    kls = None
    if seed % 2:
        kls = [o + n if rng.random() < 0.6 else int(rng.integers(1, o + n + 1)) for o in offsets]
    window = None if seed == 0 else int(rng.integers(1, 300))
    _check(n, offsets, kls, window)


def test_size_query_and_errors():
    import ctypes as C
    mt = C.c_int32()
    offs = (C.c_int32 * 2)(7, 2)
    assert vkv.lib().vkv_batch_causal_mask(4, offs, None, 2, -1, None, C.c_int64(0), None,
                                           C.byref(mt)) == 0 and mt.value == 11
    buf = torch.empty(2 * 4 * 11 - 1, dtype=torch.uint8, device="cuda")
    assert vkv.lib().vkv_batch_causal_mask(4, offs, None, 2, -1, C.c_void_p(buf.data_ptr()),
                                           C.c_int64(buf.numel()), None, C.byref(mt)) == 1
    assert b"fewer than" in vkv.lib().vkv_last_error()
    assert vkv.lib().vkv_batch_causal_mask(4, offs, None, 0, -1, None, C.c_int64(0), None,
                                           C.byref(mt)) == 1
    assert b"at least one sequence" in vkv.lib().vkv_last_error()


def test_batched_step_through_the_mask():
    rng = np.random.default_rng(7)
    dtype, B, Hq, Hkv, D, n = O.BF16, 5, 8, 2, 128, 6
    offsets = [0, 37, 120, 9, 64]
    lens = [o + n for o in offsets]
    total = max(lens)
    q = rand_bits(rng, (B, Hq, n, D), dtype)
    k = rand_bits(rng, (B, Hkv, total, D), dtype)
    v = rand_bits(rng, (B, Hkv, total, D), dtype)
    for b, L in enumerate(lens):  # padding is zeros
        k[b, :, L:] = 0
        v[b, :, L:] = 0
    mask = vkv.batch_causal_mask(n, offsets, window_size=50)
    out = vkv.scaled_dot_product_attention(dev(q, dtype), dev(k, dtype), dev(v, dtype), D ** -0.5,
                                           mask=mask)
    got = values(out, dtype)
    f = lambda a: O.to_f32(a, dtype)
    for b, L in enumerate(lens):
        m = R.causal_mask(n, offsets[b], 50)[None, None]
        ref = O.sdpa(f(q[b:b + 1]), f(k[b:b + 1, :, :L]), f(v[b:b + 1, :, :L]), D ** -0.5,
                     mask=m, q_dtype=dtype)
        assert (np.abs(got[b:b + 1] - ref) <= attn_tol(dtype, ref)).all(), b
