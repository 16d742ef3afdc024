"""GPU parity of the fixed-buffer device-offset caches (CompilableKVCache,
CompilableRotatingKVCache) and the dynamic slice ops through the C ABI
against oracle/kvcache_ref.py: buffers, masks, state, metaState and
counters are bit-exact; attention over the whole buffer with the cache's
mask agrees with attention over the plain cache; and a decode step (update,
mask, attention) captured once in a HIP graph replays correctly, each replay
checked against the same step run eagerly."""
import numpy as np
import pytest
import torch

import kvcache_ref as R
import oracle as O
import vkv
from gpu_util import attn_tol, dev, host, rand_bits, values

pytestmark = pytest.mark.gpu


def npv(a):
    return host(vkv.to_torch(a))


@pytest.mark.parametrize("dtype", [O.BF16, O.F32])
def test_dynamic_slice_update_and_slice(dtype):
    rng = np.random.default_rng(3)
    for shape, axis in [((2, 3, 40, 16), 2), ((5, 33), 1), ((64,), 0), ((4, 9, 7), 0)]:
        dst_np = rand_bits(rng, shape, dtype)
        n = max(1, shape[axis] // 4)
        us = list(shape)
        us[axis] = n
        upd_np = rand_bits(rng, tuple(us), dtype)
        for start in [0, 3, shape[axis] - n, shape[axis] + 5, -2]:
            d = dev(dst_np, dtype)
            st = torch.tensor([start], dtype=torch.int32, device="cuda")
            vkv.dynamic_slice_update(d, dev(upd_np, dtype), st, axis)
            exp = R.dynamic_slice_update_ref(dst_np, upd_np, start, axis)
            assert np.array_equal(host(d), exp), (shape, axis, start)
            sl = vkv.dynamic_slice(d, st, axis, n)
            assert np.array_equal(host(sl), R.dynamic_slice_ref(exp, start, axis, n))


def test_dynamic_slice_update_strided_source():
    rng = np.random.default_rng(4)
    big = rand_bits(rng, (2, 4, 3, 8), O.BF16)
    src = dev(big, O.BF16)[:, ::2]          # [2, 2, 3, 8], strided heads
    dst_np = np.zeros((2, 2, 10, 8), np.uint16)
    d = dev(dst_np, O.BF16)
    vkv.dynamic_slice_update(d, src, torch.tensor([6], dtype=torch.int32, device="cuda"), 2)
    exp = R.dynamic_slice_update_ref(dst_np, big[:, ::2], 6, 2)
    assert np.array_equal(host(d), exp)


def test_compilable_update_mask_state_match_oracle():
    dtype, M = O.BF16, 64
    rng = np.random.default_rng(11)
    s = vkv.KVCacheSimple()
    k = rand_bits(rng, (2, 4, 37, 32), dtype)
    v = rand_bits(rng, (2, 4, 37, 16), dtype)
    s.update(dev(k, dtype), dev(v, dtype))
    c = vkv.CompilableKVCache.from_cache(s, max_length=M)
    r = R.CompilableKVCacheRef.from_state([k, v], M)
    assert c.offset == 37 and c.capacity == M
    for n in [1, 1, 3, 1, 2, 1]:
        for window in (None, 5):
            m = c.make_mask(n, window)
            assert np.array_equal(host(m), r.make_mask(n, window)), (n, window)
        k1 = rand_bits(rng, (2, 4, n, 32), dtype)
        v1 = rand_bits(rng, (2, 4, n, 16), dtype)
        ok, ov = c.update(dev(k1, dtype), dev(v1, dtype))
        rk, rv = r.update(k1, v1)
        assert ok.shape[2] == M and ov.shape[2] == M
        assert np.array_equal(npv(ok), rk) and np.array_equal(npv(ov), rv)
        assert c.offset == r.offset
    st = c.state
    assert np.array_equal(host(st[0]), r.state[0]) and np.array_equal(host(st[1]), r.state[1])
    assert c.trim(4) == 4 and c.offset == r.offset - 4
    inner = c.inner_state()
    assert len(inner) == 3 and inner[0].shape[2] == M and inner[2].shape[0] == 1
    assert int(host(vkv.to_torch(inner[2]))[0]) == r.offset - 4


def test_compilable_snapshot_copy():
    """CompilableKVCacheSnapshotTests.swift:20-71: a copy is a snapshot."""
    def make(offset):
        c = vkv.CompilableKVCache(max_length=64)
        z = torch.zeros((1, 2, 4, 8), dtype=torch.float32, device="cuda")
        c.update(z, z)
        c.offset = offset
        return c

    c = make(12)
    snap = c.copy()
    assert snap.offset == 12
    c.offset = 40
    assert c.offset == 40 and snap.offset == 12
    c = make(30)
    snap = c.copy()
    assert c.trim(10) == 10 and c.offset == 20 and snap.offset == 30
    c = make(0)
    snap = c.copy()
    before = float(snap.state[0].sum()) if snap.state else 0.0
    one = torch.ones((1, 2, 4, 8), dtype=torch.float32, device="cuda")
    c.update(one, one)
    after = float(snap.state[0].sum()) if snap.state else 0.0
    assert before == after


@pytest.mark.parametrize("max_size,keep", [(16, 0), (16, 2)])
def test_compilable_rotating_promotion_and_wrap(max_size, keep):
    dtype = O.F16
    rng = np.random.default_rng(max_size * 10 + keep)
    rot = vkv.RotatingKVCache(max_size, keep=keep)
    ref = R.RotatingKVCacheRef(max_size, keep)
    for _ in range(10):
        k1 = rand_bits(rng, (1, 4, 1, 16), dtype)
        v1 = rand_bits(rng, (1, 4, 1, 16), dtype)
        rot.update(dev(k1, dtype), dev(v1, dtype))
        ref.update(k1, v1)
    c = vkv.CompilableRotatingKVCache.from_rotating(rot)
    cr = R.CompilableRotatingKVCacheRef.from_rotating(ref)
    # CompilableRotatingKVCacheTests.swift:57-78
    assert c.offset == 10
    inner = c.inner_state()
    assert len(inner) == 4 and inner[0].shape[2] == max_size
    assert inner[2].shape[0] == 1 and inner[3].shape[0] == 1
    for step in range(30):
        for window in (None, 6):
            assert np.array_equal(host(c.make_mask(1, window)), cr.make_mask(1, window)), step
        k1 = rand_bits(rng, (1, 4, 1, 16), dtype)
        v1 = rand_bits(rng, (1, 4, 1, 16), dtype)
        ok, ov = c.update(dev(k1, dtype), dev(v1, dtype))
        rk, rv = cr.update(k1, v1)
        assert np.array_equal(npv(ok), rk) and np.array_equal(npv(ov), rv), step
    assert c.offset == cr.offset
    assert c.meta_state == [str(keep), str(max_size), "256", str(cr.offset), str(cr.idx)]
    assert not c.is_trimmable


def test_compilable_attention_matches_plain_cache():
    """Attention over the whole fixed buffer with the cache's mask equals
    attention over the plain cache's returned keys (and the oracle)."""
    dtype, M, D = O.BF16, 256, 64
    rng = np.random.default_rng(21)
    s = vkv.KVCacheSimple()
    k = rand_bits(rng, (1, 4, 100, D), dtype)
    v = rand_bits(rng, (1, 4, 100, D), dtype)
    s.update(dev(k, dtype), dev(v, dtype))
    c = vkv.CompilableKVCache.from_cache(s, max_length=M)
    for step in range(5):
        k1 = rand_bits(rng, (1, 4, 1, D), dtype)
        v1 = rand_bits(rng, (1, 4, 1, D), dtype)
        q = dev(rand_bits(rng, (1, 16, 1, D), dtype), dtype)
        mask = c.make_mask(1)
        ck, cv = c.update(dev(k1, dtype), dev(v1, dtype))
        sk, sv = s.update(dev(k1, dtype), dev(v1, dtype))
        a = vkv.scaled_dot_product_attention(q, ck, cv, D ** -0.5, mask=mask)
        b = vkv.scaled_dot_product_attention(q, sk, sv, D ** -0.5)
        ref = O.sdpa(O.to_f32(host(q), dtype), O.to_f32(npv(sk), dtype), O.to_f32(npv(sv), dtype),
                     D ** -0.5)
        tol = attn_tol(dtype, ref)
        assert (np.abs(values(a, dtype) - ref) <= tol).all(), step
        assert (np.abs(values(b, dtype) - values(a, dtype)) <= tol).all(), step


def test_compiled_decode_step_graph_replay():
    """update + makeMask + attention captured once in a HIP graph, replayed
    six times with new inputs copied in between; every replay equals the same
    step run eagerly on a twin cache, and the device offset advances."""
    dtype, M, D, Hkv, Hq = O.BF16, 128, 64, 2, 8
    rng = np.random.default_rng(31)
    pre_k = rand_bits(rng, (1, Hkv, 20, D), dtype)
    pre_v = rand_bits(rng, (1, Hkv, 20, D), dtype)

    def fresh():
        s = vkv.KVCacheSimple()
        s.update(dev(pre_k, dtype), dev(pre_v, dtype))
        return vkv.CompilableKVCache.from_cache(s, max_length=M)

    cap, twin = fresh(), fresh()
    kin = torch.zeros((1, Hkv, 1, D), dtype=torch.bfloat16, device="cuda")
    vin = torch.zeros_like(kin)
    qin = torch.zeros((1, Hq, 1, D), dtype=torch.bfloat16, device="cuda")
    out = torch.empty((1, Hq, 1, D), dtype=torch.bfloat16, device="cuda")

    def step(cache, o):
        mask = cache.make_mask(1)
        ck, cv = cache.update(kin, vin)
        vkv.scaled_dot_product_attention(qin, ck, cv, D ** -0.5, mask=mask, out=o)

    # nothing may allocate under capture: warm the capture stream's
    # attention workspace on a throwaway cache and make the captured cache's
    # mask buffer first
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        warm = fresh()
        step(warm, torch.empty_like(out))
        cap.make_mask(1)
    torch.cuda.synchronize()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            step(cap, out)
    torch.cuda.synchronize()
    # capture records without running: the captured cache has not moved
    assert cap.offset == 20
    for r in range(6):
        kin.copy_(dev(rand_bits(rng, (1, Hkv, 1, D), dtype), dtype))
        vin.copy_(dev(rand_bits(rng, (1, Hkv, 1, D), dtype), dtype))
        qin.copy_(dev(rand_bits(rng, (1, Hq, 1, D), dtype), dtype))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        eager = torch.empty_like(out)
        step(twin, eager)
        torch.cuda.synchronize()
        assert torch.equal(out, eager), r
        assert cap.offset == twin.offset == 21 + r
    kc, vc = cap.state
    kt, vt = twin.state
    assert torch.equal(kc, kt) and torch.equal(vc, vt)


def _paged_scene(rng, n_seqs, L, Hkv=8, D=128, bs=32, bits=4):
    nb = n_seqs * ((L + bs - 1) // bs) + 1
    pool = vkv.PagedPool(nb, bs, 1, Hkv, D, dtype=vkv.BF16, bits=bits)
    tab = (1 + np.arange(n_seqs * ((L + bs - 1) // bs), dtype=np.int32)).reshape(n_seqs, -1)
    slots = [int(tab[s, p // bs]) * bs + p % bs for s in range(n_seqs) for p in range(L)]
    k = rand_bits(rng, (n_seqs * L, Hkv, D), O.BF16)
    v = rand_bits(rng, (n_seqs * L, Hkv, D), O.BF16)
    pool.append(0, dev(k, O.BF16), dev(v, O.BF16),
                torch.tensor(slots, dtype=torch.int32, device="cuda"))
    tab_dev = torch.from_numpy(tab).cuda()
    lens = torch.full((n_seqs,), L, dtype=torch.int32, device="cuda")
    return pool, pool.view(0, tab_dev, lens, L), (tab_dev, lens)


def test_workspace_growth_after_capture_keeps_graph_valid():
    """A paged decode step captured in a graph keeps the stream workspace
    address it was captured with.  A larger eager call on the same stream
    then grows the workspace; the outgrown buffer must stay allocated, so
    later replays still equal the eager result.  Growth during a capture is
    refused with an error instead of allocating."""
    rng = np.random.default_rng(41)
    D, Hq = 128, 32
    small = _paged_scene(rng, 4, 1500)
    big = _paged_scene(rng, 48, 700)
    q_small = dev(rand_bits(rng, (4, Hq, D), O.BF16), O.BF16)
    q_big = dev(rand_bits(rng, (48, Hq, D), O.BF16), O.BF16)
    out = torch.empty((4, Hq, D), dtype=torch.bfloat16, device="cuda")
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    print("workspace: warm + capture", flush=True)
    with torch.cuda.stream(s):
        vkv.paged_attention(q_small, small[1], D ** -0.5, out=torch.empty_like(out))
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            vkv.paged_attention(q_small, small[1], D ** -0.5, out=out)
    torch.cuda.synchronize()
    want = vkv.paged_attention(q_small, small[1], D ** -0.5)
    print("workspace: grow on the capture stream", flush=True)
    with torch.cuda.stream(s):
        big_out = vkv.paged_attention(q_big, big[1], D ** -0.5)
    torch.cuda.synchronize()
    assert torch.equal(big_out, vkv.paged_attention(q_big, big[1], D ** -0.5))
    for r in range(3):
        out.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, want), r
    # growth under capture: a fresh stream has no workspace yet
    s2 = torch.cuda.Stream()
    g2 = torch.cuda.CUDAGraph()
    print("workspace: growth under capture is refused", flush=True)
    with pytest.raises(vkv.VKVError, match="graph capture"):
        with torch.cuda.stream(s2):
            with torch.cuda.graph(g2, stream=s2):
                vkv.paged_attention(q_small, small[1], D ** -0.5, out=out)
    torch.cuda.synchronize()
    del g
    torch.cuda.synchronize()
    assert vkv.workspace_release(s) > 0
