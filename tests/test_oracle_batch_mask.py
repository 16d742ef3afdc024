"""The batch mask restatement (createBatchCausalMask,
BatchEngine/BatchMask.swift:44-115) pinned two ways: the reference's own
known answers (BatchEngineTests.swift:163-231 and :360-394,
CacheCoordinatorTopologyFocusedTests.swift:1613-1636), and, for unwrapped
slots, the composition it is defined by -- each slot's createCausalMask
row block (KVCache.swift:314-336, itself pinned against the compilable
cache) padded with false to the longest key length, as
BatchKVCache.padAndConcatenate pads the keys (BatchKVCache.swift:177-193)."""
import numpy as np
import pytest

import kvcache_ref as R


def test_reference_known_answers():
    m = R.batch_causal_mask(1, [5, 3])
    assert m.shape == (2, 1, 1, 6)
    assert m[0, 0, 0].tolist() == [True] * 6
    assert m[1, 0, 0].tolist() == [True] * 4 + [False] * 2
    m = R.batch_causal_mask(1, [5, 3], window=3)
    assert m[0, 0, 0, 2:6].tolist() == [False, True, True, True]
    assert m[1, 0, 0, 0:4].tolist() == [False, True, True, True]
    m = R.batch_causal_mask(1, [4, 4])
    assert m.shape == (2, 1, 1, 5) and m.all()
    m = R.batch_causal_mask(3, [2])
    assert m.shape == (1, 1, 3, 5)
    assert m[0, 0, 0, 2] and not m[0, 0, 0, 3] and m[0, 0, 2].all()
    # a wrapped ring slot beside an unbounded one
    m = R.batch_causal_mask(1, [100, 5], key_lens=[16, 6])
    assert m.shape == (2, 1, 1, 16)
    assert m[0, 0, 0].all()
    assert m[1, 0, 0].tolist() == [True] * 6 + [False] * 10
    # the same through BatchKVCache.makeMask's key lengths (ring of 16 after
    # 40 tokens, a simple cache at 5), window = maxSize
    m = R.batch_causal_mask(1, [40, 5], key_lens=[16, 6], window=16)
    assert m[0, 0, 0].all() and m[1, 0, 0].tolist() == [True] * 6 + [False] * 10


@pytest.mark.parametrize("seed", range(6))
def test_unwrapped_slots_are_padded_causal_masks(seed):
    rng = np.random.default_rng(seed)
    B = int(rng.integers(1, 7))
    n = int(rng.integers(0, 6))
    offsets = [int(x) for x in rng.integers(0, 40, B)]
    window = None if seed % 2 else int(rng.integers(1, 12))
    m = R.batch_causal_mask(n, offsets, window=window)
    total = max(o + n for o in offsets)
    assert m.shape == (B, 1, n, total)
    for b, off in enumerate(offsets):
        single = R.causal_mask(n, off, window)
        want = np.zeros((n, total), bool)
        want[:, : off + n] = single
        assert np.array_equal(m[b, 0], want), (b, off, n, window)
    # shorter key lengths than offset + n on some slots: those are wrapped
    kls = [o + n if b % 2 else min(o + n, 9) for b, o in enumerate(offsets)]
    m = R.batch_causal_mask(n, offsets, key_lens=kls, window=window)
    for b, (off, kl) in enumerate(zip(offsets, kls)):
        row = np.arange(m.shape[-1]) < kl
        if kl < off + n:
            assert np.array_equal(m[b, 0], np.broadcast_to(row, (n, m.shape[-1])))
