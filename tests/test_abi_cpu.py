"""CPU checks of the C-ABI library: it loads without a GPU, exports every
symbol include/vkv.h declares, reports errors the mlx-c way, and its host
logic (chain hash, prefix-cache manager) matches the reference.

The prefix-manager scenarios restate Tests/MLXLMTests/PagedCacheTests.swift
(:8-186) against the C ABI (no pool attached: pure host bookkeeping), and a
randomized differential test compares it with the Python restatement in
oracle/kvcache_ref.py.
"""
import ctypes as C
import os
import random
import re

import pytest

import kvcache_ref as R
import vkv

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_symbols():
    text = open(os.path.join(ROOT, "include", "vkv.h")).read()
    return sorted(set(re.findall(r"^(?:int|const char \*)\s*(vkv_\w+)\s*\(", text, re.M)))


def test_library_exports_every_declared_symbol():
    L = vkv.lib()
    decl = declared_symbols()
    assert len(decl) >= 45
    missing = [s for s in decl if not hasattr(L, s)]
    assert not missing
    assert sorted(vkv.EXPORTS) == decl
    assert L.vkv_abi_version() == 2


def test_errors_are_reported_not_thrown():
    L = vkv.lib()
    p = vkv.CacheParams(99, 0, 0, 0, 0, 0)
    h = C.c_void_p()
    assert L.vkv_cache_create(C.byref(p), C.byref(h)) == 1
    assert b"unknown cache kind" in L.vkv_last_error()
    with pytest.raises(vkv.VKVError, match="maxSize"):
        vkv.RotatingKVCache(0)
    q = vkv.QuantizedKVCache(64, 4)
    with pytest.raises(vkv.VKVError, match="updateQuantized"):  # KVCache.swift:1126-1130
        vkv._chk(L.vkv_cache_update(q._h, None, None, None, None, None))
    # CompilableTurboQuantKVCache(from:) needs a compressed source
    # (CompilableTurboQuantKVCache.swift:111-112)
    tq = vkv.TurboQuantKVCache()
    assert L.vkv_turboquant_to_compilable(tq._h, None, C.byref(h)) == 1
    assert b"compressed phase" in L.vkv_last_error()
    # the last error is per thread and cleared by the next success
    assert L.vkv_abi_version() == 2


def test_meta_state_roundtrip_and_validation():
    r = vkv.RotatingKVCache(max_size=16, keep=4, step=8)
    assert r.meta_state == ["4", "16", "8", "0", "0"]
    r.meta_state = ["4", "16", "8", "20", "9"]
    assert r.offset == 20 and r.meta_state[4] == "9"
    with pytest.raises(vkv.VKVError, match="maxSize=None"):
        r.meta_state = ["4", "None", "8", "20", "9"]
    with pytest.raises(vkv.VKVError, match="exactly 5"):
        r.meta_state = ["1"]
    s = vkv.KVCacheSimple()
    assert s.meta_state == [""]
    with pytest.raises(vkv.VKVError, match="no meta_state"):
        s.meta_state = ["x"]
    q = vkv.QuantizedKVCache(64, 4)
    assert q.meta_state == ["256", "0", "64", "4"]
    q.meta_state = ["256", "37", "64", "4"]
    assert q.offset == 37
    q.meta_state = ["256", "junk", "64", "4"]
    assert q.offset == 0  # Int(...) ?? 0 (KVCache.swift:1175)


def test_trim_bookkeeping_without_data():
    s = vkv.KVCacheSimple()
    assert s.is_trimmable and s.trim(5) == 0
    r = vkv.RotatingKVCache(max_size=8)
    assert r.is_trimmable and r.max_size == 8
    r.meta_state = ["0", "8", "256", "9", "1"]
    assert not r.is_trimmable  # offset >= maxSize (KVCache.swift:855-857)


# ------------------------------------------------------------ chain hash
@pytest.mark.parametrize("parent,key,salt", [(None, None, None), ("ab" * 32, None, None),
                                             (None, "model-x", None), (None, None, "img"),
                                             ("cd" * 32, "m", "s")])
def test_block_hash_matches_hashlib(parent, key, salt):
    toks = [1, 2, 3, -7, 2 ** 40, 0]
    assert vkv.block_hash(parent, toks, key, salt) == R.block_hash(parent, toks, key, salt)
    assert len(vkv.block_hash(parent, toks, key, salt)) == 64


def test_block_hash_properties():
    """CacheBlockTests.swift:6-70: determinism, parent / salt / key separation."""
    t = [1, 2, 3, 4, 5]
    a = vkv.block_hash(None, t)
    assert a == vkv.block_hash(None, t)
    assert vkv.block_hash("abc", t) != vkv.block_hash("xyz", t)
    p1, p2 = vkv.block_hash(None, [10, 20]), vkv.block_hash(None, [10, 21])
    assert vkv.block_hash(p1, [30, 40]) != vkv.block_hash(p2, [30, 40])
    assert a != vkv.block_hash(None, t, media_salt="imageA")
    assert vkv.block_hash(None, t, "model-x", "imageA") != vkv.block_hash(None, t, "model-y", "imageA")


# ------------------------------------------------------- PagedCacheTests
def test_paged_cache_allocation_and_free():  # PagedCacheTests.swift:8-25
    m = vkv.PagedCacheManager(block_size=4, max_blocks=8)
    b = m.allocate_block()
    assert b is not None and b != 0 and m.ref_count(b) == 1
    assert m.stats["allocated_blocks"] == 1 and m.stats["free_blocks"] == 6
    m.free_block(b)
    assert m.stats["allocated_blocks"] == 0 and m.stats["free_blocks"] == 7


def test_paged_cache_exhaustion():  # :27-50
    m = vkv.PagedCacheManager(block_size=4, max_blocks=4)
    got = [m.allocate_block() for _ in range(3)]
    assert None not in got
    assert m.allocate_block() is None and m.stats["free_blocks"] == 0
    m.free_block(got[0])
    assert m.stats["free_blocks"] == 1
    assert m.allocate_block() == got[0]


def test_paged_cache_prefix_match():  # :52-75
    m = vkv.PagedCacheManager(block_size=4, max_blocks=20)
    m.store_token_sequence(list(range(1, 11)), n_data_chunks=2)
    r = m.fetch_prefix(list(range(1, 13)))
    assert r is not None
    matched, remaining, blocks = r
    assert matched == 8 and remaining == [9, 10, 11, 12] and len(blocks) == 2


def test_paged_cache_partial_match():  # :77-97
    m = vkv.PagedCacheManager(block_size=4, max_blocks=20)
    m.store_token_sequence(list(range(1, 9)), n_data_chunks=2)
    matched, remaining, blocks = m.fetch_prefix([1, 2, 3, 4, 99, 98, 97, 96, 10, 11, 12, 13])
    assert matched == 4 and remaining == [99, 98, 97, 96, 10, 11, 12, 13] and len(blocks) == 1


def test_paged_cache_reuses_stored_partial_leaf():  # :99-122
    m = vkv.PagedCacheManager(block_size=4, max_blocks=20)
    m.store_token_sequence([1, 2, 3, 4, 5, 6], n_data_chunks=2)
    matched, remaining, blocks = m.fetch_prefix([1, 2, 3, 4, 5, 6, 7, 8])
    assert matched == 6 and remaining == [7, 8] and len(blocks) == 2
    m.free_block(blocks[1])
    m.free_block(blocks[0])


def test_paged_cache_miss():  # :124-140
    m = vkv.PagedCacheManager(block_size=4, max_blocks=20)
    m.store_token_sequence(list(range(1, 9)), n_data_chunks=2)
    assert m.fetch_prefix([99, 98, 97, 96, 95, 94, 93, 92]) is None
    assert m.stats["cache_misses"] > 0


def test_paged_cache_tiny_pool_keeps_usable_prefix():  # :142-158
    m = vkv.PagedCacheManager(block_size=2, max_blocks=2)
    m.store_token_sequence([1, 2, 3, 4, 5, 6], n_data_chunks=3)
    matched, remaining, blocks = m.fetch_prefix([1, 2, 3, 4, 5, 6, 7])
    assert matched == 2 and remaining == [3, 4, 5, 6, 7] and len(blocks) == 1


def test_paged_cache_releases_leaves_before_roots():  # :160-186
    m = vkv.PagedCacheManager(block_size=2, max_blocks=4, model_key="leaf-first-release")
    original = [1, 2, 3, 4, 5, 6]
    m.store_token_sequence(original, n_data_chunks=3)
    matched, _, blocks = m.fetch_prefix(original)
    m.release(blocks)  # CacheCoordinator.release(blocks:): leaves first
    m.store_token_sequence([9, 10], n_data_chunks=1)
    matched, remaining, _ = m.fetch_prefix(original)
    assert matched == 4 and remaining == [5, 6]


def test_sentinel_never_allocated_and_register_find():
    m = vkv.PagedCacheManager(block_size=4, max_blocks=5)
    ids = [m.allocate_block() for _ in range(5)]
    assert 0 not in ids and ids[4] is None and sorted(ids[:4]) == [1, 2, 3, 4]
    h = vkv.block_hash(None, [7, 7])
    m.register_block(ids[0], h)
    assert m.find_cached_block(h) == ids[0]
    assert m.find_cached_block("00" * 32) is None
    m.clear()
    assert m.stats["free_blocks"] == 4 and m.find_cached_block(h) is None


def test_prefix_manager_matches_restatement_randomized():
    rng = random.Random(11)
    for trial in range(30):
        bs, mb = rng.choice([2, 3, 4]), rng.randint(3, 12)
        key = rng.choice([None, "k"])
        a = vkv.PagedCacheManager(bs, mb, key)
        b = R.PagedCacheManagerRef(bs, mb, key)
        vocab = [1, 2, 3]
        held = []
        for step in range(40):
            op = rng.random()
            toks = [rng.choice(vocab) for _ in range(rng.randint(1, 10))]
            salt = rng.choice([None, None, "img"])
            if op < 0.45:
                nd = rng.randint(0, 5)
                a.store_token_sequence(toks, nd, media_salt=salt)
                b.store_token_sequence(toks, nd, media_salt=salt)
            elif op < 0.8:
                ra = a.fetch_prefix(toks, media_salt=salt)
                rb = b.fetch_prefix(toks, media_salt=salt)
                assert ra == (None if rb is None else (rb[0], rb[1], rb[2]))
                if ra:
                    held.extend(ra[2])
            elif held and op < 0.9:
                x = held.pop(rng.randrange(len(held)))
                a.free_block(x)
                b.free_block(x)
            elif held:
                # copy-on-write of a held block, as before a write into it
                i = rng.randrange(len(held))
                wa, wb = a.writable(held[i]), b.writable(held[i])
                assert wa == wb, (trial, step)
                if wa is not None:
                    held[i] = wa
            assert a.stats == b.stats, (trial, step)
            for x in set(held):
                assert a.ref_count(x) == b.blocks[x].ref


def _desc(shape, dtype, addr=0x1000):
    """A vkv_array descriptor with a placeholder device address (never
    dereferenced: these calls fail validation before any launch)."""
    a = vkv.Array()
    a.data = C.c_void_p(addr)
    a.dtype = dtype
    a.ndim = len(shape)
    st = 1
    for i in reversed(range(len(shape))):
        a.shape[i] = shape[i]
        a.strides[i] = st
        st *= shape[i]
    return a


def _qsdpa_args(B=2, Hq=8, Hkv=2, L=1, T=40, D=128, bits=4, g=64, dt=2):
    q = _desc((B, Hq, L, D), dt)
    k = [_desc((B, Hkv, T, D * bits // 32), 3), _desc((B, Hkv, T, D // g), dt),
         _desc((B, Hkv, T, D // g), dt)]
    v = [_desc((B, Hkv, T, D * bits // 32), 3), _desc((B, Hkv, T, D // g), dt),
         _desc((B, Hkv, T, D // g), dt)]
    out = _desc((B, Hq, L, D), dt)
    return q, k, v, out


def _call_qsdpa(q, k, v, out, bits=4):
    L = vkv.lib()
    return L.vkv_quantized_sdpa(C.byref(q), *[C.byref(x) for x in k + v], 64, bits,
                                C.c_float(0.1), 0, None, C.byref(out), None)


@pytest.mark.parametrize("case", [
    "out_heads", "out_len", "out_dim", "out_dtype", "v_batch", "v_heads", "k_scales_T",
    "v_biases_heads", "biases_dtype", "codes_dtype", "k_scales_last", "v_codes_last", "gqa",
])
def test_quantized_sdpa_rejects_mismatched_tuples(case):
    """Every tuple array must be [B, Hkv, T, .] with the right last dim and
    dtype, and out [B, Hq, L, D] in q's dtype; a mismatch is an error return
    before any device work (no GPU needed)."""
    q, k, v, out = _qsdpa_args()
    bad = {
        "out_heads": lambda: setattr_shape(out, 1, 4),
        "out_len": lambda: setattr_shape(out, 2, 3),
        "out_dim": lambda: setattr_shape(out, 3, 64),
        "out_dtype": lambda: setattr(out, "dtype", 1),
        "v_batch": lambda: setattr_shape(v[0], 0, 1),
        "v_heads": lambda: setattr_shape(v[0], 1, 4),
        "k_scales_T": lambda: setattr_shape(k[1], 2, 39),
        "v_biases_heads": lambda: setattr_shape(v[2], 1, 1),
        "biases_dtype": lambda: setattr(k[2], "dtype", 0),
        "codes_dtype": lambda: setattr(k[0], "dtype", 2),
        "k_scales_last": lambda: setattr_shape(k[1], 3, 4),
        "v_codes_last": lambda: setattr_shape(v[0], 3, 32),
        "gqa": lambda: [setattr_shape(x, 1, 3) for x in k + v],
    }[case]
    bad()
    assert _call_qsdpa(q, k, v, out) == 1
    msg = vkv.lib().vkv_last_error()
    # a validation message, not a failed device call
    assert b"must" in msg and b"device" not in msg and b"hip" not in msg, msg


def setattr_shape(a, i, n):
    a.shape[i] = n


def test_noalloc_scratch_limit_is_checked_on_the_host():
    """The no-allocation decode entry point is declared and exported; its
    argument checks are the allocating call's (a NULL view fails)."""
    L = vkv.lib()
    q = _desc((1, 8, 128), 2)
    out = _desc((1, 8, 128), 2)
    assert L.vkv_paged_sdpa_noalloc(C.byref(q), None, C.c_float(0.1), C.byref(out), None) == 1
    assert b"kv is NULL" in L.vkv_last_error()


def test_prefix_writable_copy_on_write_rules():
    """vkv_prefix_writable: a block held once and uncached is written in
    place; a forked block (refcount 2) or a cached block (a fetched prefix
    leaf) moves the caller to a fresh block; an exhausted pool gives None."""
    m = vkv.PagedCacheManager(4, 6)
    b = m.allocate_block()
    assert m.writable(b) == b and m.ref_count(b) == 1
    m.incref(b)  # forked to a second sequence
    c = m.writable(b)
    assert c not in (None, b) and m.ref_count(b) == 1 and m.ref_count(c) == 1
    # a stored and fetched sequence: its partial leaf is cached
    m2 = vkv.PagedCacheManager(4, 6)
    m2.store_token_sequence([1, 2, 3, 4, 5, 6], 2)
    matched, rest, blocks = m2.fetch_prefix([1, 2, 3, 4, 5, 6, 7])
    assert matched == 6 and len(blocks) == 2 and m2.ref_count(blocks[1]) == 1
    leaf = blocks[1]
    w = m2.writable(leaf)
    assert w != leaf and m2.ref_count(leaf) == 0 and m2.token_count(leaf) == 2
    # the cached leaf is still found by a later fetch
    again = m2.fetch_prefix([1, 2, 3, 4, 5, 6])
    assert again[0] == 6 and again[2][1] == leaf
    # exhaust the pool: no copy possible
    m3 = vkv.PagedCacheManager(4, 3)
    x, y = m3.allocate_block(), m3.allocate_block()
    m3.incref(x)
    assert m3.allocate_block() is None and m3.writable(x) is None and m3.ref_count(x) == 2
