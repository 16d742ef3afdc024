"""Pins of RotatingKVCacheRef (oracle/kvcache_ref.py, the restatement of
KVCache.swift:605-958) by a brute-force model that never looks at ring
indices: every token is its own absolute position, and the model keeps the
list of positions the cache must still hold.

  * a multi-token update (updateConcat, :658-680) keeps the `keep` prefix and
    the newest max_size - 1 - keep older tokens, then appends all S new ones
    ("every token gets at least maxCacheSize context", :668-671);
  * a one-token update keeps the prefix and the newest max_size - 1 - keep
    older tokens once the cache is full (the in-place write at :755-769, or
    the concat fallback chosen by canUpdateInPlace, :780-789), else appends;
  * the arrays an update returns hold exactly those tokens: in temporal
    order after a concat, in ring order (the first `offset` slots while the
    ring is not full, :764-768) after an in-place write;
  * the single-token window mask (:905-923), built before the update, marks
    visible exactly the returned keys whose position is within `window` of
    the query (absolute position = the offset before the update).  This
    holds for keep = 0, the configuration the reference's models use
    (Gemma3Text.swift:412-415).  With keep > 0 the reference rolls the mask
    over the whole ring as if the ring restarted at slot 0, while its writes
    restart at slot `keep`, so the mask is off by the prefix; the
    restatement (and the device cache) keep that behaviour, and the test
    below records it.
"""
import numpy as np
import pytest

import kvcache_ref as R


def _model_update(held, offset, S, max_size, keep):
    new = list(range(offset, offset + S))
    if not held:
        return new
    pre, rest = held[:keep], held[keep:]
    room = max_size - 1 - keep
    if S == 1 and len(held) < max_size:
        return held + new
    return pre + rest[max(0, len(rest) - room):] + new


PLANS = [
    [20] + [1] * 40 + [7] + [1] * 70 + [30] + [1] * 5,
    [1] * 130 + [3] + [1] * 60,
    [64, 1, 1, 5, 1, 17, 1, 1, 1] + [1] * 90 + [2, 2, 2] + [1] * 40,
]


@pytest.mark.parametrize("keep", [0, 4])
@pytest.mark.parametrize("plan", range(len(PLANS)))
@pytest.mark.parametrize("step", [16, 256])
def test_rotating_ref_matches_brute_force(keep, plan, step):
    max_size, window = 48, 32
    r = R.RotatingKVCacheRef(max_size, keep, step)
    held, offset = [], 0
    for i, S in enumerate(PLANS[plan]):
        tok = np.arange(offset, offset + S, dtype=np.int64).reshape(1, 1, S, 1)
        mask = r.make_mask(S, window=window) if S == 1 else None
        rk, rv = r.update(tok, tok + 1000000)
        ids = rk[0, 0, :, 0].tolist()
        held = _model_update(held, offset, S, max_size, keep)
        # returned length and content (:671-679, :764-768)
        assert len(ids) == len(held), (i, len(ids), len(held))
        assert sorted(ids) == sorted(held), i
        assert np.array_equal(rv[0, 0, :, 0], rk[0, 0, :, 0] + 1000000)
        if S > 1:
            assert ids == held, i  # temporal order after a concat
        elif offset + 1 <= max_size:
            assert ids == held, i  # no wrap yet: slots 0..offset in order
        # temporal order = keep prefix, then the newest tokens, oldest first
        tk, _ = r.temporally_ordered()
        assert tk[0, 0, :, 0].tolist() == held, i
        if S == 1 and keep == 0:
            # the query at absolute position `offset` sees keys within the window
            want = np.array([p >= offset - window + 1 for p in ids])
            if isinstance(mask, str):
                assert mask == "none" and want.all(), i
            else:
                assert np.array_equal(np.asarray(mask, bool), want), i
        offset += S
        assert r.offset == offset


def test_rotating_ref_rolled_mask_after_wrap():
    """A window narrower than the ring after several wraps: the rolled mask
    keeps exactly the newest `window` keys visible (:905-923)."""
    max_size, window = 40, 8
    r = R.RotatingKVCacheRef(max_size, 0, 16)
    for offset in range(3 * max_size + 7):
        tok = np.full((1, 1, 1, 1), offset, np.int64)
        mask = r.make_mask(1, window=window)
        rk, _ = r.update(tok, tok)
        ids = rk[0, 0, :, 0]
        vis = ids >= offset - window + 1
        if isinstance(mask, str):
            assert vis.all()
        else:
            assert np.array_equal(np.asarray(mask, bool), vis)
            assert int(np.asarray(mask, bool).sum()) == window


def test_rotating_ref_mask_with_keep_prefix_is_the_unshifted_roll():
    """keep > 0: after the ring wraps, the reference's mask is the window
    over absolute positions of a ring that restarts at slot 0, i.e. it
    differs from the window over the tokens actually held."""
    max_size, window, keep = 48, 32, 4
    r = R.RotatingKVCacheRef(max_size, keep, 16)
    differs = 0
    for offset in range(3 * max_size):
        tok = np.full((1, 1, 1, 1), offset, np.int64)
        mask = r.make_mask(1, window=window)
        rk, _ = r.update(tok, tok)
        if isinstance(mask, str):
            continue
        ids = rk[0, 0, :, 0]
        m = np.asarray(mask, bool)
        assert int(m.sum()) == window
        differs += not np.array_equal(m, ids >= offset - window + 1)
    assert differs > 0
