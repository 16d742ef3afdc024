"""CPU checks of the TurboQuant host side (no device memory is touched):
the library's EncoderState tables -- rotation signs, Lloyd-Max codebooks,
QJL matrix -- are bit-exact with the restatement (oracle.tq_*, pinned in
test_oracle_turboquant.py) for several (dim, bits, seed);
hasCompressibleMiddle (TurboQuantKVCache.swift:152-162); the cache's
construction defaults and argument errors."""
import ctypes as C

import numpy as np
import pytest

import oracle as O
import vkv


@pytest.mark.parametrize("dim,bits,seed", [(128, 2, 42), (128, 3, 42), (64, 1, 7), (16, 2, 0),
                                           (192, 4, 42), (100, 3, 5), (256, 3, 42)])
def test_tables_match_the_restatement(dim, bits, seed):
    signs, cb, S = vkv.tq_tables(dim, bits, seed)
    assert np.array_equal(signs, O.tq_random_signs(dim, seed))
    assert np.array_equal(cb, O.tq_codebook(dim, bits))
    assert np.array_equal(S, O.tq_qjl_matrix(dim, seed + 1000))


@pytest.mark.parametrize("tokens,sink,res,minimum,want", [
    (76, 4, 64, 8, True), (75, 4, 64, 8, False), (3, 4, 64, 8, False), (10, 0, 0, 8, True),
    (10, -3, -1, 8, True), (100, 4, 200, 1, False), (0, 4, 64, 0, True), (9, 1, 0, 8, True)])
def test_has_compressible_middle(tokens, sink, res, minimum, want):
    assert vkv.TurboQuantKVCache.has_compressible_middle(tokens, sink, res, minimum) is want


def test_create_defaults_and_errors():
    c = vkv.TurboQuantKVCache()
    assert c.info == {"phase": 0, "has_encoded": 0, "prefix_tokens": 0, "window_tokens": 0,
                      "key_bits": 3, "value_bits": 3, "sink_tokens": 4, "residual_tokens": 64}
    assert c.offset == 0 and c.is_trimmable and c.meta_state == [""]
    c.meta_state = ["ignored"]  # the setter ignores its value
    c2 = vkv.TurboQuantKVCache(2, 4, 0, -5)
    assert c2.info["residual_tokens"] == 0
    for kb, vb in ((0, 3), (10, 3), (3, 0), (3, 9)):
        with pytest.raises(vkv.VKVError, match="Bits must be in"):
            vkv.TurboQuantKVCache(kb, vb)
    k, v = vkv.TQEncoded(), vkv.TQEncoded()
    assert vkv.lib().vkv_turboquant_encoded(c._h, C.byref(k), C.byref(v)) == 1
    assert b"no encoded record" in vkv.lib().vkv_last_error()
    params = vkv.CacheParams(vkv.CACHE_TURBOQUANT, 0, 0, 0, 0, 4)
    h = C.c_void_p()
    assert vkv.lib().vkv_cache_create(C.byref(params), C.byref(h)) == 0
    t = vkv.TurboQuantKVCache(handle=h)
    assert t.info["key_bits"] == 4 and t.info["value_bits"] == 4
