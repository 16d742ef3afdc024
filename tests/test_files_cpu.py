"""CPU checks of the on-disk formats (no device memory is touched): the
DiskCache file-name hash against hashlib, and the prompt-cache / disk-record
readers' validation of files written here by an independent safetensors
writer (the `safetensors` package) in the reference's layout
(KVCache.swift:1620-1845, TQDiskSerializer.swift:15-103): unknown classes,
count mismatches, RotatingKVCache maxSize None, malformed containers and
disk records with a gap in their layer kinds all fail before any cache is
built, with the reference's messages."""
import ctypes as C
import hashlib
import json
import os
import struct

import numpy as np
import pytest
from safetensors.numpy import save_file

import vkv


def test_disk_hash_matches_hashlib():
    """DiskCache.hashTokens (DiskCache.swift:659-682): model key, then
    "|media:" + salt, then the tokens as little-endian Int64; 32 hex."""
    toks = [1, 2, 3, 70000, -5, 2 ** 40]
    raw = struct.pack("<%dq" % len(toks), *toks)
    for key, salt in [(None, None), ("qwen", None), ("qwen", "img0"), (None, "s")]:
        h = hashlib.sha256()
        if key is not None:
            h.update(key.encode())
        if salt is not None:
            h.update(b"|media:" + salt.encode())
        h.update(raw)
        assert vkv.disk_hash_tokens(toks, key, salt) == h.hexdigest()[:32]
    assert vkv.disk_hash_tokens([]) == hashlib.sha256(b"").hexdigest()[:32]


def _load_count(path):
    n = C.c_int32()
    nm = C.c_int32()
    rc = vkv.lib().vkv_prompt_cache_load(path.encode(), None, None, 0, C.byref(n), None,
                                         C.c_int64(0), C.byref(nm))
    return rc, n.value, nm.value, vkv.lib().vkv_last_error().decode()


def _prompt_file(path, classes, infos, n_arrays=2, extra_meta=None):
    arrays = {}
    for i in range(n_arrays):
        arrays[f"{i}.0"] = np.zeros((1, 2, 3, 8), np.float32)
        arrays[f"{i}.1"] = np.zeros((1, 2, 3, 8), np.float32)
    meta = {}
    for i, info in enumerate(infos):
        for j, v in enumerate(info):
            meta[f"0.{i}.{j}"] = v
    for i, c in enumerate(classes):
        meta[f"2.{i}"] = c
    meta.update(extra_meta or {})
    save_file(arrays, path, metadata=meta)


def test_prompt_cache_reader_counts_and_metadata(tmp_path):
    p = str(tmp_path / "ok.safetensors")
    _prompt_file(p, ["KVCache", "RotatingKVCache"], [[""], ["0", "64", "256", "70", "6"]],
                 extra_meta={"1.model": "m", "1.a.b": "dotted key"})
    rc, n, nm, err = _load_count(p)
    assert rc == 0 and n == 2 and nm == 2, err
    buf = C.create_string_buffer(256)
    n2, nm2 = C.c_int32(), C.c_int32()
    assert vkv.lib().vkv_prompt_cache_load(p.encode(), None, None, 0, C.byref(n2), buf, C.c_int64(256),
                                           C.byref(nm2)) == 0
    parts = buf.raw.split(b"\0")[:4]
    assert dict(zip(parts[::2], parts[1::2])) == {b"model": b"m", b"a.b": b"dotted key"}
    assert vkv.lib().vkv_prompt_cache_load(p.encode(), None, None, 0, C.byref(n2), buf, C.c_int64(5),
                                           C.byref(nm2)) == 1
    assert b"too small" in vkv.lib().vkv_last_error()


@pytest.mark.parametrize("case,message", [
    ("unknown_class", "Unknown cache class: MambaCacheX"),
    ("count_mismatch", "Mismatch in cache counts"),
    ("rotating_none", "maxSize=None is not supported"),
    ("rotating_short", "expected 5 values"),
    ("rotating_bad", "Failed to parse RotatingKVCache maxSize"),
])
def test_prompt_cache_reader_errors(tmp_path, case, message):
    """loadPromptCache's errors (KVCache.swift:1703-1762)."""
    p = str(tmp_path / f"{case}.safetensors")
    if case == "unknown_class":
        _prompt_file(p, ["KVCache", "MambaCacheX"], [[""], [""]])
    elif case == "count_mismatch":
        _prompt_file(p, ["KVCache"], [[""], [""]])
    elif case == "rotating_none":
        _prompt_file(p, ["RotatingKVCache", "KVCache"], [["0", "None", "256", "0", "0"], [""]])
    elif case == "rotating_short":
        _prompt_file(p, ["RotatingKVCache", "KVCache"], [["0", "64"], [""]])
    else:
        _prompt_file(p, ["RotatingKVCache", "KVCache"], [["0", "sixty", "256", "0", "0"], [""]])
    rc, n, nm, err = _load_count(p)
    assert rc == 1 and message in err, err


def _raw_file(path, header: dict, data: bytes, pad=True):
    h = json.dumps(header).encode()
    if pad:
        h += b" " * ((8 - (8 + len(h)) % 8) % 8)
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(h)) + h + data)


@pytest.mark.parametrize("case,message", [
    ("offsets_past_end", "do not fit"),
    ("offsets_wrong_size", "do not fit"),
    ("bad_dtype", "unsupported dtype"),
    ("header_too_long", "header length"),
    ("not_json", "safetensors header"),
    ("float_offset", "non-integer"),
    ("missing_file", "cannot open"),
    # dims each within bounds whose product wraps int64 to 0 (2^32 * 2^32)
    ("shape_overflow", "too large"),
])
def test_safetensors_container_validation(tmp_path, case, message):
    p = str(tmp_path / f"{case}.safetensors")
    meta = {"__metadata__": {"2.0": "KVCache", "0.0.0": ""}}
    ent = lambda off, dt="F32", shape=(1, 2, 3, 8): {"dtype": dt, "shape": list(shape),
                                                     "data_offsets": list(off)}
    data = bytes(4 * 48)
    if case == "offsets_past_end":
        _raw_file(p, {**meta, "0.0": ent((0, 192)), "0.1": ent((192, 384))}, data)
    elif case == "offsets_wrong_size":
        _raw_file(p, {**meta, "0.0": ent((0, 100)), "0.1": ent((100, 192))}, data)
    elif case == "bad_dtype":
        _raw_file(p, {**meta, "0.0": ent((0, 192), "C64"), "0.1": ent((0, 192))}, data)
    elif case == "header_too_long":
        with open(p, "wb") as f:
            f.write(struct.pack("<Q", 10 ** 9) + b"{}")
    elif case == "not_json":
        with open(p, "wb") as f:
            f.write(struct.pack("<Q", 8) + b"{\"a\": [}")
    elif case == "float_offset":
        h = {**meta, "0.0": {"dtype": "F32", "shape": [1, 2, 3, 8], "data_offsets": [0.0, 192]}}
        _raw_file(p, h, data)
    elif case == "shape_overflow":
        _raw_file(p, {**meta, "0.0": ent((0, 0), shape=(1, 1, 2 ** 32, 2 ** 32)),
                      "0.1": ent((0, 192))}, data)
    if case != "missing_file":
        assert os.path.exists(p)
    rc, n, nm, err = _load_count(p)
    assert rc == 1 and message in err, err


def test_disk_record_reader_counts_and_required_miss(tmp_path):
    """deserializeV2 (TQDiskSerializer.swift:1023-1070): the layer count is
    the highest kind tag + 1; a gap in the tags is a required miss, as is a
    kind this library does not hold; version 1 records are refused."""
    i32 = lambda v: np.array([v], np.int32)
    kv = np.zeros((1, 2, 3, 8), np.float32)
    good = {"__jang_cache_format_version__": i32(2), "__tq_native_marker__": i32(1),
            "__layer_kind_0__": i32(2), "kv_0_keys": kv, "kv_0_values": kv,
            "__layer_kind_1__": i32(4)}
    p = str(tmp_path / "good.safetensors")
    save_file(good, p, metadata={"format": "mlx"})
    n = C.c_int32()
    assert vkv.lib().vkv_disk_cache_load(p.encode(), None, None, 0, C.byref(n)) == 0 and n.value == 2
    cases = {
        "gap": {**good, "__layer_kind_3__": i32(2)},
        "tq": {**good, "__layer_kind_1__": i32(1)},
        "v1": {k: v for k, v in good.items() if k != "__jang_cache_format_version__"},
        "incomplete": {k: v for k, v in good.items() if k != "kv_0_values"},
    }
    want = {"gap": "no kind tag", "tq": "required miss", "v1": "version-2",
            "incomplete": "incomplete kv payload"}
    for name, arrays in cases.items():
        q = str(tmp_path / f"{name}.safetensors")
        save_file(arrays, q, metadata={"format": "mlx"})
        hs = (C.c_void_p * 8)()
        rc = vkv.lib().vkv_disk_cache_load(q.encode(), None, hs if name != "v1" else None, 8,
                                           C.byref(n))
        if name in ("gap", "tq", "incomplete"):
            # the count pass succeeds; building the caches refuses the record
            # before any layer is restored
            assert rc == 1 and want[name] in vkv.lib().vkv_last_error().decode(), name
            assert all(h is None for h in hs), name
        else:
            assert rc == 1 and want[name] in vkv.lib().vkv_last_error().decode(), name


def _tq_record(window_values=True, offset=100):
    """A kind-1 layer in serializeTQLayer's layout (TQDiskSerializer.swift:
    368-429) with 28 encoded + 4 sink + 64 tail tokens and a 4-token
    window (zeros: only the structure is read before the check fails)."""
    i32 = lambda *v: np.array(v, np.int32)
    f16 = lambda *s: np.zeros(s, np.float16)
    words = lambda n, bits: np.zeros(-(-n // (32 // bits)), np.uint32)
    n = 4 * 28 * 16
    rec = {"__jang_cache_format_version__": i32(2), "__layer_kind_0__": i32(1),
           "tq_0_ck_indices": words(n, 3), "tq_0_ck_qjl": words(n, 1),
           "tq_0_ck_res_norms": f16(1, 4, 28, 1), "tq_0_ck_vec_norms": f16(1, 4, 28, 1),
           "tq_0_ck_sink": f16(1, 4, 4, 16), "tq_0_ck_tail": f16(1, 4, 64, 16),
           "__tq_0_ck_shape__": i32(1, 4, 28, 16), "__tq_0_ck_index_bits__": i32(3),
           "__tq_0_ck_seed__": i32(42), "tq_0_cv_indices": words(n, 4),
           "tq_0_cv_norms": f16(1, 4, 28, 1), "tq_0_cv_sink": f16(1, 4, 4, 16),
           "tq_0_cv_tail": f16(1, 4, 64, 16), "__tq_0_cv_shape__": i32(1, 4, 28, 16),
           "__tq_0_cv_index_bits__": i32(4), "__tq_0_cv_seed__": i32(42),
           "__tq_0_offset__": i32(offset), "tq_0_window_keys": f16(1, 4, offset - 96, 16)}
    if window_values:
        rec["tq_0_window_values"] = f16(1, 4, offset - 96, 16)
    return rec


@pytest.mark.parametrize("case,message", [
    ("missing_window_values", "missing TurboQuant window"),
    ("short_offset", "inconsistent TurboQuant token counts"),
    ("no_qjl", "incomplete TurboQuant payload"),
    ("unexpected_window", "unexpected TurboQuant window"),
])
def test_disk_record_turboquant_required_misses(tmp_path, case, message):
    """deserializeTQLayer's refusals (TQDiskSerializer.swift:1244-1346) and
    the reference test that drops tq_0_window_values
    (TQDiskSerializerTests.swift:221-239): the whole record is refused
    before any layer is built."""
    rec = _tq_record()
    if case == "missing_window_values":
        rec = _tq_record(window_values=False)
    elif case == "short_offset":
        rec["__tq_0_offset__"] = np.array([90], np.int32)
    elif case == "no_qjl":
        del rec["tq_0_ck_qjl"]
    elif case == "unexpected_window":
        rec["__tq_0_offset__"] = np.array([96], np.int32)
    p = str(tmp_path / f"{case}.safetensors")
    save_file(rec, p, metadata={"format": "mlx"})
    n = C.c_int32()
    hs = (C.c_void_p * 4)()
    assert vkv.lib().vkv_disk_cache_load(p.encode(), None, hs, 4, C.byref(n)) == 1
    err = vkv.lib().vkv_last_error().decode()
    assert message in err and "required miss" in err, err
    assert all(h is None for h in hs)
