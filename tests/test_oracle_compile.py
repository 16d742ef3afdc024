"""Pins of the oracle's restatement of the fixed-buffer caches and dynamic
slices (oracle/kvcache_ref.py) by independent formulations, on the CPU:
element-wise definitions of the slice ops, the simple cache's state and the
createCausalMask function for CompilableKVCache, a brute-force ring for
CompilableRotatingKVCache, and the reference's own scenario expectations
(CompilableKVCacheSnapshotTests.swift:20-71,
CompilableRotatingKVCacheTests.swift:57-78)."""
import numpy as np
import pytest

import kvcache_ref as R


def test_dynamic_slice_update_elementwise():
    rng = np.random.default_rng(0)
    for shape, axis in [((3, 17), 1), ((2, 3, 9, 4), 2), ((11,), 0), ((5, 6, 7), 0)]:
        dst = rng.integers(0, 1000, shape)
        n = max(1, shape[axis] // 3)
        ushape = list(shape)
        ushape[axis] = n
        upd = rng.integers(1000, 2000, ushape)
        for start in [0, 1, shape[axis] - n, shape[axis] - n + 2, -3, 10 ** 6]:
            got = R.dynamic_slice_update_ref(dst, upd, start, axis)
            s = min(max(start, 0), shape[axis] - n)
            exp = dst.copy()
            for idx in np.ndindex(*shape):
                p = idx[axis]
                if s <= p < s + n:
                    src = list(idx)
                    src[axis] = p - s
                    exp[idx] = upd[tuple(src)]
            assert np.array_equal(got, exp), (shape, axis, start)
            sl = R.dynamic_slice_ref(got, start, axis, n)
            assert np.array_equal(sl, upd)


def test_compilable_matches_simple_cache_and_causal_mask():
    rng = np.random.default_rng(1)
    L, M = 37, 64
    k = rng.integers(0, 60000, (2, 3, L, 8)).astype(np.uint16)
    v = rng.integers(0, 60000, (2, 3, L, 5)).astype(np.uint16)
    s = R.KVCacheSimpleRef()
    s.update(k, v)
    c = R.CompilableKVCacheRef.from_state(s.state, M)
    assert c.offset == L and c.keys.shape[2] == M
    for step, n in enumerate([1, 1, 3, 1, 2]):
        for window in (None, 4):
            m = c.make_mask(n, window)
            cm = R.causal_mask(n, c.offset, window)
            assert np.array_equal(m[:, :c.offset + n], cm)
            assert not m[:, c.offset + n:].any()
        k1 = rng.integers(0, 60000, (2, 3, n, 8)).astype(np.uint16)
        v1 = rng.integers(0, 60000, (2, 3, n, 5)).astype(np.uint16)
        rk, rv = s.update(k1, v1)
        ck, cv = c.update(k1, v1)
        assert ck.shape[2] == M and c.offset == s.offset
        assert np.array_equal(ck[:, :, :c.offset], rk) and np.array_equal(cv[:, :, :c.offset], rv)
        assert not ck[:, :, c.offset:].any()
        assert all(np.array_equal(a, b) for a, b in zip(c.state, s.state))


def test_compilable_snapshot_expectations():
    # CompilableKVCacheSnapshotTests.swift:20-71: offset set to 12 / 30, copy,
    # later writes and trims do not reach the copy
    c = R.CompilableKVCacheRef(64)
    c.update(np.zeros((1, 2, 4, 8), np.float32), np.zeros((1, 2, 4, 8), np.float32))
    c.offset = 30
    snap = R.CompilableKVCacheRef.from_state([c.keys, c.values], 64)
    snap.offset = c.offset
    assert c.trim(10) == 10 and c.offset == 20 and snap.offset == 30


@pytest.mark.parametrize("max_size,keep", [(16, 0), (16, 3), (7, 1)])
def test_compilable_rotating_ring_brute_force(max_size, keep):
    """Token t (1-based) written at step t lands in the slot a brute-force
    ring gives: slots [0, keep) hold the first keep tokens for good, the
    rest cycle through [keep, max_size)."""
    r = R.RotatingKVCacheRef(max_size, keep)
    pre = 5
    for t in range(1, pre + 1):
        r.update(np.full((1, 1, 1, 2), t, np.int64), np.full((1, 1, 1, 2), t, np.int64))
    c = R.CompilableRotatingKVCacheRef.from_rotating(r)
    # promotion (CompilableRotatingKVCacheTests.swift:57-78)
    assert c.offset == pre and c.keys.shape[2] == max_size
    ring = [0] * max_size
    for t in range(1, pre + 1):
        ring[t - 1] = t
    ptr = pre  # next slot of a plain ring that skips the kept slots
    for t in range(pre + 1, pre + 3 * max_size):
        c.update(np.full((1, 1, 1, 2), t, np.int64), np.full((1, 1, 1, 2), t, np.int64))
        if ptr == max_size:
            ptr = keep
        ring[ptr] = t
        ptr += 1
        assert list(c.keys[0, 0, :, 0]) == ring, t
        assert c.offset == t
        m = c.make_mask(1)
        assert m.all() if t >= max_size else (m[0] == (np.arange(max_size) <= t)).all()
    # once full, the ring holds the first keep tokens and the newest
    # max_size - keep ones, as the rotating cache's temporal order does
    held = sorted(c.keys[0, 0, :, 0].tolist())
    last = pre + 3 * max_size - 1
    exp = list(range(1, keep + 1)) + list(range(last - (max_size - keep) + 1, last + 1))
    assert held == sorted(exp)
