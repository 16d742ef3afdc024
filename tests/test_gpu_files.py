"""GPU round trips of the on-disk formats, with the files read back by an
independent safetensors implementation (the `safetensors` package):

  * savePromptCache / loadPromptCache (KVCache.swift:1620-1845) for a
    KVCacheSimple (f16), a wrapped RotatingKVCache (bf16) and a 4-bit
    QuantizedKVCache: the file's tensor names "i.j", metadata "0.i.j",
    "1.<key>", "2.i" and bytes equal the caches' state; loading restores
    class, offset, metaState and state bit-exact; a file written by the
    independent writer in the same layout loads into equal caches;
  * the disk tier's version-2 record (TQDiskSerializer.swift) for the same
    three layers plus an empty one (kind 4);
  * the prompt-cache file from / into pool blocks: a 4-bit pool sequence
    saved, loaded as QuantizedKVCache objects (state = the pool's codes),
    and loaded into a second 4-bit pool (codes bit-exact), an 8-bit pool
    (requantized: the oracle quantizer of the dequantized values) and a
    bf16 pool (the dequantized values)."""
import numpy as np
import pytest
import torch
from safetensors import safe_open
from safetensors.torch import save_file

import oracle as O
import vkv
from gpu_util import dev, host, rand_bits

pytestmark = pytest.mark.gpu


def _caches(rng):
    simple = vkv.KVCacheSimple()
    k = rand_bits(rng, (1, 2, 300, 64), O.F16)
    v = rand_bits(rng, (1, 2, 300, 64), O.F16)
    simple.update(dev(k, O.F16), dev(v, O.F16))
    rot = vkv.RotatingKVCache(64, keep=0, step=16)
    for t in range(100):  # past a wrap: the ring order and idx are saved
        x = rand_bits(rng, (2, 2, 1, 64), O.BF16)
        rot.update(dev(x, O.BF16), dev(x, O.BF16))
    q = vkv.QuantizedKVCache(64, 4)
    q.update_quantized(dev(rand_bits(rng, (1, 4, 70, 128), O.BF16), O.BF16),
                       dev(rand_bits(rng, (1, 4, 70, 128), O.BF16), O.BF16))
    return [simple, rot, q]


def _state_np(c):
    return [x.detach().contiguous().cpu() for x in c.state]


def _raw(t):
    """Shape and bytes of a CPU tensor (u32 codes read as int32 or uint32)."""
    t = t.contiguous()
    if t.dtype in (torch.bfloat16, torch.float16):
        t = t.view(torch.int16)
    elif t.dtype == torch.uint32:
        t = t.view(torch.int32)
    return tuple(t.shape), t.numpy().tobytes()


def _same_state(a, b):
    sa, sb = _state_np(a), _state_np(b)
    assert len(sa) == len(sb)
    for x, y in zip(sa, sb):
        assert x.dtype == y.dtype and _raw(x) == _raw(y)


def test_prompt_cache_round_trip_and_layout(tmp_path):
    rng = np.random.default_rng(80)
    caches = _caches(rng)
    path = str(tmp_path / "prompt.safetensors")
    vkv.save_prompt_cache(path, caches, {"model": "test-model", "step": "7"})
    with safe_open(path, framework="pt") as f:
        meta = f.metadata()
        names = sorted(f.keys())
        tensors = {k: f.get_tensor(k) for k in names}
    assert names == sorted(["0.0", "0.1", "1.0", "1.1"] + [f"2.{j}" for j in range(6)])
    assert meta["2.0"] == "KVCache" and meta["2.1"] == "RotatingKVCache"
    assert meta["2.2"] == "QuantizedKVCache"
    assert meta["1.model"] == "test-model" and meta["1.step"] == "7"
    for i, c in enumerate(caches):
        ms = c.meta_state
        for j, s in enumerate(ms):
            assert meta[f"0.{i}.{j}"] == s
        for j, x in enumerate(_state_np(c)):
            assert _raw(tensors[f"{i}.{j}"]) == _raw(x), (i, j)
    assert tensors["2.0"].dtype == torch.uint32  # the codes are stored as U32
    loaded, user = vkv.load_prompt_cache(path)
    assert user == {"model": "test-model", "step": "7"}
    for a, b in zip(caches, loaded):
        assert type(a) is type(b) and a.offset == b.offset and a.meta_state == b.meta_state
        _same_state(a, b)
    # the restored caches keep working: one more update on the rotating one
    x = dev(rand_bits(rng, (2, 2, 1, 64), O.BF16), O.BF16)
    ka, _ = caches[1].update(x, x)
    kb, _ = loaded[1].update(x, x)
    assert torch.equal(vkv.to_torch(ka).cpu(), vkv.to_torch(kb).cpu())


def test_prompt_cache_written_by_another_writer_loads(tmp_path):
    """A file in the reference's layout from an independent writer."""
    rng = np.random.default_rng(81)
    k = torch.from_numpy(rand_bits(rng, (1, 2, 40, 64), O.BF16).view(np.int16)).view(torch.bfloat16)
    v = torch.from_numpy(rand_bits(rng, (1, 2, 40, 64), O.BF16).view(np.int16)).view(torch.bfloat16)
    path = str(tmp_path / "other.safetensors")
    save_file({"0.0": k, "0.1": v}, path, metadata={"0.0.0": "", "2.0": "KVCache", "1.x": "y"})
    (c,), user = vkv.load_prompt_cache(path)
    assert user == {"x": "y"} and isinstance(c, vkv.KVCacheSimple) and c.offset == 40
    sk, sv = _state_np(c)
    assert torch.equal(sk.view(torch.int16), k.view(torch.int16))
    assert torch.equal(sv.view(torch.int16), v.view(torch.int16))


def test_disk_record_round_trip(tmp_path):
    rng = np.random.default_rng(82)
    caches = _caches(rng) + [vkv.KVCacheSimple()]
    path = str(tmp_path / (vkv.disk_hash_tokens([1, 2, 3], "m") + ".safetensors"))
    vkv.disk_cache_save(path, caches)
    with safe_open(path, framework="pt") as f:
        meta = f.metadata()
        t = {k: f.get_tensor(k) for k in f.keys()}
    assert meta == {"format": "mlx"}
    assert t["__jang_cache_format_version__"].tolist() == [2]
    assert [t[f"__layer_kind_{i}__"].tolist() for i in range(4)] == [[2], [6], [5], [4]]
    assert t["__rot_1_meta__"].tolist() == [int(s) for s in caches[1].meta_state]
    assert t["__qkv_2_count__"].tolist() == [6] and t["__qkv_2_bits__"].tolist() == [4]
    assert t["__qkv_2_group_size__"].tolist() == [64] and t["__qkv_2_offset__"].tolist() == [70]
    loaded = vkv.disk_cache_load(path)
    assert len(loaded) == 4 and loaded[3] is None
    for a, b in zip(caches[:3], loaded[:3]):
        assert type(a) is type(b) and a.offset == b.offset and a.meta_state == b.meta_state
        _same_state(a, b)


def _pool_with_sequence(rng, bits, dtype=vkv.BF16, n=100, bs=32, H=2, D=128, nblk=12):
    pool = vkv.PagedPool(nblk, bs, 2, H, D, dtype=dtype, bits=bits)
    blocks = [int(b) for b in rng.permutation(np.arange(1, nblk))[: (n + bs - 1) // bs]]
    slots = torch.tensor([blocks[p // bs] * bs + p % bs for p in range(n)], dtype=torch.int32,
                         device="cuda")
    kv = []
    for layer in range(2):
        k = rand_bits(rng, (n, H, D), O.BF16, outliers=2)
        v = rand_bits(rng, (n, H, D), O.BF16, outliers=2)
        pool.append(layer, dev(k, O.BF16), dev(v, O.BF16), slots)
        kv.append((k, v))
    return pool, blocks, kv


def _view(pool, layer, blocks, n):
    tab = torch.tensor([blocks], dtype=torch.int32, device="cuda")
    return pool.view(layer, tab, torch.tensor([n], dtype=torch.int32, device="cuda"), n)


def test_prompt_cache_from_and_into_pool_blocks(tmp_path):
    rng = np.random.default_rng(83)
    n = 100
    pool, blocks, kv = _pool_with_sequence(rng, 4)
    path = str(tmp_path / "paged.safetensors")
    vkv.save_prompt_cache_paged(path, pool, blocks, n, {"seq": "1"})
    # as cache objects: QuantizedKVCache layers holding the pool's codes
    caches, user = vkv.load_prompt_cache(path)
    assert user == {"seq": "1"} and len(caches) == 2
    for layer, c in enumerate(caches):
        assert isinstance(c, vkv.QuantizedKVCache) and c.offset == n
        assert c.meta_state == ["256", str(n), "64", "4"]
        (kq, ks, kb), (vq, vs, vb) = vkv.paged_gather_quantized(_view(pool, layer, blocks, n))
        for got, want in zip(c.state, (kq, ks, kb, vq, vs, vb)):
            assert _raw(got.cpu()) == _raw(want[0:1].cpu())
    # into pools of three formats
    for bits, dtype in ((4, vkv.BF16), (8, vkv.BF16), (0, vkv.BF16)):
        p2 = vkv.PagedPool(16, 32, 2, 2, 128, dtype=dtype, bits=bits)
        blocks2 = [5, 9, 2, 14]
        nt, meta = vkv.load_prompt_cache_paged(path, p2, blocks2)
        assert nt == n and meta == {"seq": "1"}
        for layer in range(2):
            k, v = kv[layer]
            src = [np.ascontiguousarray(x.transpose(1, 0, 2)) for x in (k, v)]  # [H, n, D]
            q4 = [O.quantize(x, O.BF16, 64, 4) for x in src]
            deq = [O.dequantize(q[0], q[1], q[2], O.BF16, 64, 4) for q in q4]
            view = _view(p2, layer, blocks2, n)
            if bits == 4:
                (kq, ks, kb), (vq, vs, vb) = vkv.paged_gather_quantized(view)
                for got, want in zip((kq, ks, kb, vq, vs, vb), q4[0][:3] + q4[1][:3]):
                    assert np.array_equal(host(got[0]).view(want.dtype), want), (bits, layer)
            elif bits == 8:
                (kq, ks, kb), (vq, vs, vb) = vkv.paged_gather_quantized(view)
                q8 = [O.quantize(d, O.BF16, 64, 8) for d in deq]
                for got, want in zip((kq, ks, kb, vq, vs, vb), q8[0][:3] + q8[1][:3]):
                    assert np.array_equal(host(got[0]).view(want.dtype), want), (bits, layer)
            else:
                kd, vd = vkv.paged_gather(view)
                assert np.array_equal(host(kd[0]), deq[0]) and np.array_equal(host(vd[0]), deq[1])
