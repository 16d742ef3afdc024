"""GPU parity of the paged block pool: append through slot mappings into
randomly permuted block tables with refcounted shared prefix blocks,
gather (raw codes bit-exact with the oracle quantizer, dequant-on-read
bit-exact with the oracle dequantizer, float blocks bit-exact), decode
attention over mixed-length sequences (tolerance vs the oracle), and the
prefix cache storing/fetching device blocks."""
import numpy as np
import pytest
import torch

import oracle as O
import vkv
from gpu_util import OPTIONS, assert_qclose, assert_within, qattn_tol, qref, attn_tol, dev, host, rand_bits, values

pytestmark = pytest.mark.gpu


class Paged:
    """A small continuous-batching scene: sequences with random block
    tables drawn from a pool, the first `n_share` sharing a prefix."""

    def __init__(self, rng, bits, dtype=O.BF16, n_seqs=6, bs=32, Hkv=8, D=128, nblocks=96,
                 share_tokens=64, n_share=3, max_len=300, lens=None):
        self.rng, self.bits, self.dtype, self.bs, self.Hkv, self.D = rng, bits, dtype, bs, Hkv, D
        self.pool = vkv.PagedPool(nblocks, bs, 1, Hkv, D, dtype=dtype, bits=bits)
        self.mgr = vkv.PagedCacheManager(bs, nblocks, pool=self.pool)
        if lens is None:
            lens = [int(x) for x in rng.integers(share_tokens + 1, max_len, n_seqs)]
            lens[-1] = 1  # a one-token sequence
        self.lens = list(lens)
        self.tokens = [rand_bits(rng, (L, Hkv, D), dtype, outliers=2) for L in self.lens]
        self.vals = [rand_bits(rng, (L, Hkv, D), dtype, outliers=2) for L in self.lens]
        n_sh_blocks = share_tokens // bs
        shared = [self.mgr.allocate_block() for _ in range(n_sh_blocks)]
        self.tables = []
        for s, L in enumerate(self.lens):
            nb = (L + bs - 1) // bs + 1  # room for a decode step
            own = [self.mgr.allocate_block() for _ in range(nb)]
            if s < n_share:
                for b in shared:
                    self.mgr.incref(b)
                own[:n_sh_blocks] = shared
                # sharing sequences see the same prefix tokens
                self.tokens[s][:share_tokens] = self.tokens[0][:share_tokens]
                self.vals[s][:share_tokens] = self.vals[0][:share_tokens]
            self.tables.append(own)
        self.share_tokens, self.n_share = share_tokens, n_share
        self.width = max(len(t) for t in self.tables)

    def slots(self, s, positions):
        return [self.tables[s][p // self.bs] * self.bs + p % self.bs for p in positions]

    def append_all(self):
        keys, vals, slots = [], [], []
        for s, L in enumerate(self.lens):
            start = self.share_tokens if 0 < s < self.n_share else 0
            keys.append(self.tokens[s][start:])
            vals.append(self.vals[s][start:])
            slots += self.slots(s, range(start, L))
        k = np.concatenate(keys)
        v = np.concatenate(vals)
        sl = torch.tensor(slots, dtype=torch.int32, device="cuda")
        self.pool.append(0, dev(k, self.dtype), dev(v, self.dtype), sl)

    def view(self):
        tab = np.full((len(self.lens), self.width), -1, np.int32)
        for s, t in enumerate(self.tables):
            tab[s, :len(t)] = t
        self.tab_dev = torch.from_numpy(tab).cuda()
        self.len_dev = torch.tensor(self.lens, dtype=torch.int32, device="cuda")
        return self.pool.view(0, self.tab_dev, self.len_dev, max(self.lens))


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("dtype", [O.BF16, O.F16])
def test_paged_quantized_append_gather_attention(bits, dtype):
    rng = np.random.default_rng(bits * 10 + dtype)
    P = Paged(rng, bits, dtype)
    P.append_all()
    view = P.view()
    (kq, ks, kb), (vq, vs, vb) = vkv.paged_gather_quantized(view)
    kd, vd = vkv.paged_gather(view)
    torch.cuda.synchronize()
    Hq, scale = 32, P.D ** -0.5
    q = rand_bits(rng, (len(P.lens), Hq, P.D), dtype)
    out = values(vkv.paged_attention(dev(q, dtype), view, scale), dtype)
    f = lambda a: O.to_f32(a, dtype)
    for s, L in enumerate(P.lens):
        for which, src, got in ((0, P.tokens[s], (kq, ks, kb)), (1, P.vals[s], (vq, vs, vb))):
            x = np.ascontiguousarray(src.transpose(1, 0, 2))  # [H, L, D]
            rq, rs, rb, _ = O.quantize(x, dtype, 64, bits)
            assert np.array_equal(host(got[0][s, :, :L]), rq), (s, which)
            assert np.array_equal(host(got[1][s, :, :L]).view(rs.dtype), rs)
            assert np.array_equal(host(got[2][s, :, :L]).view(rb.dtype), rb)
            deq = O.dequantize(rq, rs, rb, dtype, 64, bits)
            assert np.array_equal(host((kd, vd)[which][s, :, :L]), deq)
        rk = O.quantize(np.ascontiguousarray(P.tokens[s].transpose(1, 0, 2)), dtype, 64, bits)
        rv = O.quantize(np.ascontiguousarray(P.vals[s].transpose(1, 0, 2)), dtype, 64, bits)
        ref, wb = (x[0, :, 0] for x in qref(f(q[s])[None, :, None], dtype, rk[0][None], f(rk[1])[None],
                               f(rk[2])[None], rv[0][None], f(rv[1])[None], f(rv[2])[None], scale,
                               64, bits))
        assert_qclose(out[s], ref, wb, dtype, f"seq {s}")


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("group", [32, 128])
def test_paged_quantized_gather_f32_groups(bits, group):
    """Dequant-on-read of f32 affine blocks (two 16-byte stores per 8 dims)
    with groups of 32 and 128, bit-exact with the oracle dequantizer."""
    dtype = O.F32
    rng = np.random.default_rng(40 + bits + group)
    P = Paged(rng, bits, dtype, n_seqs=4, D=128)
    P.pool = vkv.PagedPool(96, P.bs, 1, P.Hkv, P.D, dtype=dtype, bits=bits, group_size=group)
    P.append_all()
    kd, vd = vkv.paged_gather(P.view())
    for s, L in enumerate(P.lens):
        for src, got in ((P.tokens[s], kd), (P.vals[s], vd)):
            x = np.ascontiguousarray(src.transpose(1, 0, 2))
            rq, rs, rb, _ = O.quantize(x, dtype, group, bits)
            assert np.array_equal(host(got[s, :, :L]), O.dequantize(rq, rs, rb, dtype, group, bits)), s


def test_paged_decode_step_crosses_block_boundary():
    dtype, bits = O.BF16, 4
    rng = np.random.default_rng(21)
    P = Paged(rng, bits, dtype, n_share=0, lens=[63, 64, 65, 1])
    P.append_all()
    # one decode token per sequence at position len
    k1 = rand_bits(rng, (4, 8, 128), dtype)
    v1 = rand_bits(rng, (4, 8, 128), dtype)
    slots = [P.slots(s, [L])[0] for s, L in enumerate(P.lens)]
    P.pool.append(0, dev(k1, dtype), dev(v1, dtype), torch.tensor(slots, dtype=torch.int32, device="cuda"))
    for s in range(4):
        P.tokens[s] = np.concatenate([P.tokens[s], k1[s:s + 1]])
        P.vals[s] = np.concatenate([P.vals[s], v1[s:s + 1]])
        P.lens[s] += 1
    view = P.view()
    (kq, ks, kb), (vq, _, _) = vkv.paged_gather_quantized(view)
    for s, L in enumerate(P.lens):
        rq = O.quantize(np.ascontiguousarray(P.vals[s].transpose(1, 0, 2)), dtype, 64, bits)[0]
        assert np.array_equal(host(vq[s, :, :L]), rq)


@pytest.mark.parametrize("dtype", [O.BF16, O.F16, O.F32])
def test_paged_float_pool(dtype):
    rng = np.random.default_rng(31 + dtype)
    P = Paged(rng, 0, dtype, n_seqs=5, bs=16)
    P.append_all()
    view = P.view()
    kd, vd = vkv.paged_gather(view)
    q = rand_bits(rng, (len(P.lens), 32, 128), dtype)
    out = values(vkv.paged_attention(dev(q, dtype), view, 0.09), dtype)
    f = (lambda a: O.to_f32(a, dtype)) if dtype != O.F32 else (lambda a: a)
    for s, L in enumerate(P.lens):
        k = np.ascontiguousarray(P.tokens[s].transpose(1, 0, 2))
        v = np.ascontiguousarray(P.vals[s].transpose(1, 0, 2))
        assert np.array_equal(host(kd[s, :, :L]), k) and np.array_equal(host(vd[s, :, :L]), v)
        ref = O.sdpa(f(q[s])[None, :, None], f(k)[None], f(v)[None], 0.09)[0, :, 0]
        assert (np.abs(out[s] - ref) <= attn_tol(dtype, ref)).all()


def test_prefix_store_fetch_copies_device_blocks():
    """storeTokenSequence copies each chunk's KV into fresh pool blocks;
    fetchPrefix returns them and a gather through them restores the KV
    (restoreLayerData, CacheHelpers.swift:431-552)."""
    dtype, bits = O.BF16, 4
    rng = np.random.default_rng(41)
    P = Paged(rng, bits, dtype, n_seqs=2, n_share=0, max_len=150)
    P.append_all()
    L = P.lens[0]
    toks = [int(x) for x in rng.integers(0, 1000, L)]
    n_chunks = (L + P.bs - 1) // P.bs
    P.mgr.store_token_sequence(toks, n_chunks, src_blocks=P.tables[0][:n_chunks])
    r = P.mgr.fetch_prefix(toks + [5, 6])
    assert r is not None
    matched, remaining, blocks = r
    assert matched == L and remaining == [5, 6] and len(blocks) == n_chunks
    assert not set(blocks) & set(P.tables[0])  # copies, not the live blocks
    tab = torch.tensor([blocks], dtype=torch.int32, device="cuda")
    lens = torch.tensor([L], dtype=torch.int32, device="cuda")
    (kq, _, _), (vq, _, _) = vkv.paged_gather_quantized(P.pool.view(0, tab, lens, L))
    rq = O.quantize(np.ascontiguousarray(P.tokens[0].transpose(1, 0, 2)), dtype, 64, bits)[0]
    assert np.array_equal(host(kq[0]), rq)
    P.mgr.release(blocks)


@pytest.mark.parametrize("bits,D,rep,bs,Hkv", [(4, 128, 4, 32, 8), (4, 64, 1, 64, 2), (8, 128, 2, 32, 4),
                                               (4, 128, 8, 64, 2), (8, 64, 16, 32, 1), (4, 128, 3, 32, 2),
                                               (8, 256, 2, 32, 2), (4, 256, 2, 64, 1), (8, 128, 5, 96, 2),
                                               (4, 64, 12, 32, 1)])
def test_paged_decode_shapes_and_partitions(bits, D, rep, bs, Hkv):
    """The matrix-core decode path across GQA factors (head groups of 4 and
    8), head dims, pool block sizes (sub-blocks of 32) and sequences long
    enough to be split into several partitions, against the oracle."""
    dtype = O.BF16
    rng = np.random.default_rng(bits * 1000 + D + rep * 7 + bs)
    lens = [5000, 31, 32, 33, 700, 0 + 1]
    nblocks = sum((L + bs - 1) // bs + 1 for L in lens) + 4
    P = Paged(rng, bits, dtype, bs=bs, Hkv=Hkv, D=D, nblocks=nblocks, n_share=0, lens=lens)
    P.append_all()
    view = P.view()
    Hq = Hkv * rep
    q = rand_bits(rng, (len(lens), Hq, D), dtype)
    out = values(vkv.paged_attention(dev(q, dtype), view, D ** -0.5), dtype)
    f = lambda a: O.to_f32(a, dtype)
    for s, L in enumerate(lens):
        rk = O.quantize(np.ascontiguousarray(P.tokens[s].transpose(1, 0, 2)), dtype, 64, bits)
        rv = O.quantize(np.ascontiguousarray(P.vals[s].transpose(1, 0, 2)), dtype, 64, bits)
        ref, wb = (x[0, :, 0] for x in qref(f(q[s])[None, :, None], dtype, rk[0][None], f(rk[1])[None],
                               f(rk[2])[None], rv[0][None], f(rv[1])[None], f(rv[2])[None],
                               D ** -0.5, 64, bits))
        assert_qclose(out[s], ref, wb, dtype, f"seq {s}")


def test_generic_and_matrix_core_paths_agree(monkeypatch):
    dtype, bits = O.BF16, 4
    rng = np.random.default_rng(77)
    P = Paged(rng, bits, dtype, n_seqs=5)
    P.append_all()
    view = P.view()
    q = dev(rand_bits(rng, (len(P.lens), 32, 128), dtype), dtype)
    fast = values(vkv.paged_attention(q, view, 0.088), dtype)
    monkeypatch.setattr(OPTIONS, "generic_attention", 1)
    slow = values(vkv.paged_attention(q, view, 0.088), dtype)
    assert np.abs(fast - slow).max() <= 2e-2


@pytest.mark.parametrize("waves", ["1", "7", "5000"])
def test_decode_wave_counts_agree(monkeypatch, waves):
    """The fewest waves (the longest ranges, each crossing many sequence and
    head segments), an odd count, and more waves than units (one unit each,
    most waves idle) give the same output within fp32 rounding of the merge
    order, and repeated launches give identical bits."""
    dtype, bits = O.BF16, 4
    rng = np.random.default_rng(91)
    P = Paged(rng, bits, dtype, n_seqs=5, n_share=2, max_len=900, nblocks=200)
    P.append_all()
    view = P.view()
    q = dev(rand_bits(rng, (len(P.lens), 32, 128), dtype), dtype)
    base = values(vkv.paged_attention(q, view, 0.088), dtype)
    monkeypatch.setattr(OPTIONS, "decode_waves", int(waves))
    got = values(vkv.paged_attention(q, view, 0.088), dtype)
    for _ in range(2):
        again = values(vkv.paged_attention(q, view, 0.088), dtype)
        assert np.array_equal(again, got)
    assert np.abs(base - got).max() <= 2e-2
    f = lambda a: O.to_f32(a, dtype)
    qh = host(q)
    for s, L in enumerate(P.lens):
        rk = O.quantize(np.ascontiguousarray(P.tokens[s].transpose(1, 0, 2)), dtype, 64, bits)
        rv = O.quantize(np.ascontiguousarray(P.vals[s].transpose(1, 0, 2)), dtype, 64, bits)
        ref, wb = (x[0, :, 0] for x in qref(f(qh[s])[None, :, None], dtype, rk[0][None], f(rk[1])[None],
                               f(rk[2])[None], rv[0][None], f(rv[1])[None], f(rv[2])[None], 0.088,
                               64, bits))
        assert_qclose(got[s], ref, wb, dtype, f"seq {s}")


def test_append_aligned_groups_ragged_and_scattered_slots():
    """One append call mixing an 8-aligned prefill run (V words assembled in
    LDS), a run starting mid-group, single tokens scattered over blocks
    (nibbles merged atomically) and skipped tokens (slot -1, and slots past
    the pool's last block, which must not be written); the gathered
    codes are bit-exact with the oracle quantizer, and tokens already in
    the touched words survive."""
    dtype, bits, bs, H, D = O.BF16, 4, 32, 4, 128
    rng = np.random.default_rng(55)
    nblocks = 12
    pool = vkv.PagedPool(nblocks, bs, 1, H, D, dtype=dtype, bits=bits)
    # sequence A: blocks 1, 2 (positions 0..40 aligned run of 41 tokens)
    # sequence B: block 3, positions 3..21 (starts mid-group)
    # sequence C..F: one token each at position 5 of blocks 4..7
    ta, tb = [1, 2], [3]
    slots = [ta[p // bs] * bs + p % bs for p in range(41)]
    slots += [tb[0] * bs + p for p in range(3, 22)]
    singles = [4 * bs + 5, 5 * bs + 5, 6 * bs + 5, 7 * bs + 5]
    slots += singles + [-1, nblocks * bs + 3, 2 ** 30]
    n = len(slots)
    k = rand_bits(rng, (n, H, D), dtype, outliers=2)
    v = rand_bits(rng, (n, H, D), dtype, outliers=2)
    # first fill the words the single tokens share, to check they survive
    pre = [4 * bs + p for p in range(8)]
    pk = rand_bits(rng, (8, H, D), dtype)
    pv = rand_bits(rng, (8, H, D), dtype)
    pre_slots = [x for x in pre if x != 4 * bs + 5]
    pool.append(0, dev(pk[:7], dtype), dev(pv[:7], dtype),
                torch.tensor(pre_slots, dtype=torch.int32, device="cuda"))
    pool.append(0, dev(k, dtype), dev(v, dtype), torch.tensor(slots, dtype=torch.int32, device="cuda"))
    # views: A (41 tokens), B positions 3..21 read as a 22-token sequence,
    # block 4 as an 8-token sequence holding the pre-filled tokens + single
    tab = torch.tensor([[1, 2], [3, 0], [4, 0]], dtype=torch.int32, device="cuda")
    lens = torch.tensor([41, 22, 8], dtype=torch.int32, device="cuda")
    (kq, ks, kb), (vq, vs, vb) = vkv.paged_gather_quantized(pool.view(0, tab, lens, 41))
    want_k = {0: (k[:41], 0), 1: (k[41:60], 3)}
    want_v = {0: (v[:41], 0), 1: (v[41:60], 3)}
    for s in (0, 1):
        for src, got in ((want_k[s], (kq, ks, kb)), (want_v[s], (vq, vs, vb))):
            x, off = src
            rq, rs, rb, _ = O.quantize(np.ascontiguousarray(x.transpose(1, 0, 2)), dtype, 64, bits)
            L = x.shape[0]
            assert np.array_equal(host(got[0][s, :, off:off + L]), rq), s
            assert np.array_equal(host(got[1][s, :, off:off + L]).view(rs.dtype), rs), s
            assert np.array_equal(host(got[2][s, :, off:off + L]).view(rb.dtype), rb), s
    # block 4: positions 0..7 = pre-filled tokens with the single token at 5
    seq_k = np.concatenate([pk[:5], k[60:61], pk[5:7]])
    seq_v = np.concatenate([pv[:5], v[60:61], pv[5:7]])
    for x, got in ((seq_k, (kq, ks, kb)), (seq_v, (vq, vs, vb))):
        rq, rs, rb, _ = O.quantize(np.ascontiguousarray(x.transpose(1, 0, 2)), dtype, 64, bits)
        assert np.array_equal(host(got[0][2, :, :8]), rq)
        assert np.array_equal(host(got[1][2, :, :8]).view(rs.dtype), rs)


def test_prefix_copy_on_write_and_lru_eviction_on_device():
    """The prefix manager wired to a device pool (PagedCacheManager.swift:
    104-376): a 72-token sequence (two full 32-token blocks and an 8-token
    partial leaf) is stored (device block copies) and fetched by two
    sequences; the one that appends copies the shared leaf first
    (vkv_prefix_writable), so the cached leaf and the other sequence keep
    their bytes.  Then, with everything released, allocation under a small
    pool evicts cached blocks leaf first.  Block ids and stats follow the
    restatement step by step; the device bytes are checked through gathers
    against the oracle quantizer."""
    import kvcache_ref as R

    rng = np.random.default_rng(91)
    dtype, bits, bs, Hkv, D, nblk = O.BF16, 4, 32, 2, 64, 12
    pool = vkv.PagedPool(nblk, bs, 1, Hkv, D, dtype=dtype, bits=bits)
    mgr = vkv.PagedCacheManager(bs, nblk, pool=pool)
    ref = R.PagedCacheManagerRef(bs, nblk)
    toks = [int(x) for x in rng.integers(0, 1000, 72)]
    kx = rand_bits(rng, (73, Hkv, D), dtype)  # 72 prompt tokens + 1 generated
    vx = rand_bits(rng, (73, Hkv, D), dtype)

    def both(fa, fb):
        a, b = fa(mgr), fb(ref)
        assert a == b and mgr.stats == ref.stats, (a, b)
        return a

    def append(blocks, positions, rows):
        slots = [blocks[p // bs] * bs + p % bs for p in positions]
        pool.append(0, dev(kx[rows], dtype), dev(vx[rows], dtype),
                    torch.tensor(slots, dtype=torch.int32, device="cuda"))

    def gather(blocks, n):
        tab = torch.tensor([blocks], dtype=torch.int32, device="cuda")
        view = pool.view(0, tab, torch.tensor([n], dtype=torch.int32, device="cuda"), n)
        (kq, ks, kb), (vq, vs, vb) = vkv.paged_gather_quantized(view)
        torch.cuda.synchronize()
        return [host(x[0]) for x in (kq, ks, kb, vq, vs, vb)]

    def expect(rows):
        out = []
        for x in (kx, vx):
            rq, rs, rb, _ = O.quantize(np.ascontiguousarray(x[rows].transpose(1, 0, 2)), dtype, 64, bits)
            out += [rq, rs.view(np.uint16), rb.view(np.uint16)]
        return out

    # sequence A computes its prompt into three private blocks, stores it
    a_blocks = [both(lambda m: m.allocate_block(), lambda r: r.allocate_block()) for _ in range(3)]
    append(a_blocks, range(72), list(range(72)))
    mgr.store_token_sequence(toks, 3, src_blocks=a_blocks)
    ref.store_token_sequence(toks, 3)
    assert mgr.stats == ref.stats
    for b in reversed(a_blocks):
        both(lambda m: m.free_block(b), lambda r: r.free_block(b))
    # sequences B and C fetch it: the same three cached blocks, the last partial
    fb = both(lambda m: m.fetch_prefix(toks + [7]), lambda r: r.fetch_prefix(toks + [7]))
    fc = both(lambda m: m.fetch_prefix(toks), lambda r: r.fetch_prefix(toks))
    assert fb[0] == fc[0] == 72 and fb[2] == fc[2]
    cached = fb[2]
    assert mgr.ref_count(cached[2]) == 2 and mgr.token_count(cached[2]) == 8
    # B appends its generated token: copy-on-write of the shared leaf
    leaf_b = both(lambda m: m.writable(cached[2]), lambda r: r.writable(cached[2]))
    assert leaf_b not in cached and mgr.ref_count(cached[2]) == 1
    b_blocks = cached[:2] + [leaf_b]
    append(b_blocks, [72], [72])
    for got, want in zip(gather(b_blocks, 73), expect(list(range(73)))):
        assert np.array_equal(got.view(want.dtype), want)
    for got, want in zip(gather(cached, 72), expect(list(range(72)))):
        assert np.array_equal(got.view(want.dtype), want)  # the cache entry kept its bytes
    # a private, uncached block is written in place
    assert both(lambda m: m.writable(leaf_b), lambda r: r.writable(leaf_b)) == leaf_b
    # release everything (leaves first), then allocate until the first
    # cached block is evicted: it is the partial leaf
    def ref_release(r, blocks):
        for x in reversed(blocks):
            r.free_block(x)

    for blocks in (b_blocks, cached):
        both(lambda m: m.release(blocks), lambda r: ref_release(r, blocks))
    taken = []
    while ref.stats["evictions"] == 0:
        taken.append(both(lambda m: m.allocate_block(), lambda r: r.allocate_block()))
        assert taken[-1] is not None
    assert taken[-1] == cached[2]
    hit = both(lambda m: m.fetch_prefix(toks), lambda r: r.fetch_prefix(toks))
    assert hit[0] == 64 and hit[2] == cached[:2]
    for got, want in zip(gather(cached[:2], 64), expect(list(range(64)))):
        assert np.array_equal(got.view(want.dtype), want)
