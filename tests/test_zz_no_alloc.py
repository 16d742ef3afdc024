"""vkv_paged_sdpa_noalloc: the decode entry point that allocates nothing
(split-K partials in the library's fixed device scratch) against
vkv_paged_sdpa on the same inputs, called through the C ABI.

Two calls in a row on the matrix-core path, the second with fewer and
shorter sequences (the scratch keeps the first call's partials, which the
second must not pick up), plus the float-block path, checked bit-exact
against the allocating entry point (same kernels, same split) and against
the oracle; an oversized call is refused before any launch."""
import numpy as np
import pytest
import torch

import oracle as O
import vkv
from gpu_util import assert_qclose, dev, host, qref, rand_bits, values

pytestmark = pytest.mark.gpu


def scene(rng, bits, lens, Hkv=8, D=128, bs=32, dtype=O.BF16):
    nblocks = sum((L + bs - 1) // bs for L in lens) + 2
    pool = vkv.PagedPool(nblocks, bs, 1, Hkv, D, dtype=dtype, bits=bits)
    perm = rng.permutation(np.arange(1, nblocks))
    tables, slots, keys, vals, i = [], [], [], [], 0
    for L in lens:
        nb = (L + bs - 1) // bs
        t = [int(b) for b in perm[i:i + nb]]
        i += nb
        tables.append(t)
        slots += [t[p // bs] * bs + p % bs for p in range(L)]
        keys.append(rand_bits(rng, (L, Hkv, D), dtype, outliers=2))
        vals.append(rand_bits(rng, (L, Hkv, D), dtype, outliers=2))
    pool.append(0, dev(np.concatenate(keys), dtype), dev(np.concatenate(vals), dtype),
                torch.tensor(slots, dtype=torch.int32, device="cuda"))
    width = max(len(t) for t in tables)
    tab = np.zeros((len(lens), width), np.int32)
    for s, t in enumerate(tables):
        tab[s, :len(t)] = t
    tab_dev = torch.from_numpy(tab).cuda()
    len_dev = torch.tensor(lens, dtype=torch.int32, device="cuda")
    view = pool.view(0, tab_dev, len_dev, max(lens))
    return pool, view, keys, vals, (tab_dev, len_dev)


def check_against_oracle(out, q, keys, vals, bits, dtype, D):
    f = lambda a: O.to_f32(a, dtype)
    for s in range(len(keys)):
        rk = O.quantize(np.ascontiguousarray(keys[s].transpose(1, 0, 2)), dtype, 64, bits)
        rv = O.quantize(np.ascontiguousarray(vals[s].transpose(1, 0, 2)), dtype, 64, bits)
        ref, wb = (x[0, :, 0] for x in qref(f(q[s])[None, :, None], dtype, rk[0][None],
                                            f(rk[1])[None], f(rk[2])[None], rv[0][None],
                                            f(rv[1])[None], f(rv[2])[None], D ** -0.5, 64, bits))
        assert_qclose(out[s], ref, wb, dtype, f"seq {s}")


@pytest.mark.parametrize("bits", [4, 8])
def test_noalloc_matches_allocating_entry_point(bits):
    rng = np.random.default_rng(700 + bits)
    dtype, Hkv, D, Hq = O.BF16, 8, 128, 32
    for call, lens in enumerate(([3000, 17, 900, 64, 2200, 1, 1500, 333], [40, 700, 5])):
        print(f"noalloc call {call}: bits {bits} lens {lens}", flush=True)
        pool, view, keys, vals, keep = scene(rng, bits, lens, Hkv, D)
        q = rand_bits(rng, (len(lens), Hq, D), dtype)
        qd = dev(q, dtype)
        want = vkv.paged_attention(qd, view, D ** -0.5)
        out = torch.empty_like(want)
        got = vkv.paged_attention(qd, view, D ** -0.5, out=out, noalloc=True)
        torch.cuda.synchronize()
        assert got.data_ptr() == out.data_ptr()
        assert np.array_equal(host(got), host(want)), call
        check_against_oracle(values(got, dtype), q, keys, vals, bits, dtype, D)


def test_noalloc_group128_matches_allocating_entry_point():
    """A group-128 cache (the matrix-core decode's group-128 mode): the
    partials merge in the merge launch here and inside the launch on the
    allocating entry point, through the same merge step in the same order,
    so the outputs are bit-identical; and within the oracle's bar."""
    from test_gpu_decode_g128 import scene as scene_g
    rng = np.random.default_rng(740)
    dtype, bits, Hkv, D, Hq = O.BF16, 4, 4, 128, 16
    lens = [1800, 40, 3300, 1]
    print(f"noalloc group 128: lens {lens}", flush=True)
    pool, view, keys, vals, keep = scene_g(rng, bits, 128, lens, Hkv, D, dtype)
    q = rand_bits(rng, (len(lens), Hq, D), dtype)
    qd = dev(q, dtype)
    want = vkv.paged_attention(qd, view, D ** -0.5)
    got = vkv.paged_attention(qd, view, D ** -0.5, out=torch.empty_like(want), noalloc=True)
    torch.cuda.synchronize()
    assert np.array_equal(host(got), host(want))
    f = lambda a: O.to_f32(a, dtype)
    out = values(got, dtype)
    for s, L in enumerate(lens):
        rk = O.quantize(np.ascontiguousarray(keys[s][:L].transpose(1, 0, 2)), dtype, 128, bits)
        rv = O.quantize(np.ascontiguousarray(vals[s][:L].transpose(1, 0, 2)), dtype, 128, bits)
        ref, wb = (x[0, :, 0] for x in qref(f(q[s])[None, :, None], dtype, rk[0][None],
                                            f(rk[1])[None], f(rk[2])[None], rv[0][None],
                                            f(rv[1])[None], f(rv[2])[None], D ** -0.5, 128, bits))
        assert_qclose(out[s], ref, wb, dtype, f"seq {s}")


def test_noalloc_float_blocks_match():
    """bf16 blocks: the generic split-K kernel, partials in the scratch."""
    rng = np.random.default_rng(710)
    dtype, Hkv, D, Hq = O.BF16, 2, 64, 8
    for call, lens in enumerate(([1800, 3, 260], [90])):
        print(f"noalloc float call {call}: lens {lens}", flush=True)
        pool, view, keys, vals, keep = scene(rng, 0, lens, Hkv, D)
        q = dev(rand_bits(rng, (len(lens), Hq, D), dtype), dtype)
        want = vkv.paged_attention(q, view, D ** -0.5)
        got = vkv.paged_attention(q, view, D ** -0.5, out=torch.empty_like(want), noalloc=True)
        torch.cuda.synchronize()
        assert np.array_equal(host(got), host(want)), call


def test_noalloc_rejects_calls_beyond_the_scratch():
    """256 sequences x 8 kv heads need 136 MB of partials at head_dim 128:
    refused with the size in the message, before anything is launched."""
    rng = np.random.default_rng(720)
    print("noalloc oversize: 256 sequences", flush=True)
    pool, view, keys, vals, keep = scene(rng, 4, [2] * 256)
    q = dev(rand_bits(rng, (256, 32, 128), O.BF16), O.BF16)
    with pytest.raises(vkv.VKVError, match="scratch"):
        vkv.paged_attention(q, view, 128 ** -0.5, out=torch.empty_like(q), noalloc=True)
    torch.cuda.synchronize()


def test_noalloc_under_graph_capture():
    """The use the entry point is for: a decode call captured in a HIP graph
    (after one eager call, which resolves the scratch on the device) and
    replayed with new queries copied in between; every replay equals the
    eager call of the allocating entry point on the same queries."""
    rng = np.random.default_rng(730)
    dtype, Hkv, D, Hq, bits = O.BF16, 8, 128, 32, 4
    lens = [1200, 31, 4000, 700]
    print(f"noalloc capture: lens {lens}", flush=True)
    pool, view, keys, vals, keep = scene(rng, bits, lens, Hkv, D)
    qin = dev(rand_bits(rng, (len(lens), Hq, D), dtype), dtype)
    out = torch.empty_like(qin)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        vkv.paged_attention(qin, view, D ** -0.5, out=out, noalloc=True)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            vkv.paged_attention(qin, view, D ** -0.5, out=out, noalloc=True)
    torch.cuda.synchronize()
    for r in range(4):
        q = rand_bits(rng, (len(lens), Hq, D), dtype)
        qin.copy_(dev(q, dtype))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        want = vkv.paged_attention(qin, view, D ** -0.5)
        torch.cuda.synchronize()
        assert np.array_equal(host(out), host(want)), r
        check_against_oracle(values(out, dtype), q, keys, vals, bits, dtype, D)
