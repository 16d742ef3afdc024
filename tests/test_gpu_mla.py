"""GPU parity of absorbed-latent MLA decode (vkv_mla_decode) against the
oracle's MLA attention (entries dequantized to bf16, fp64 softmax, values =
the first 512 dims of each 576-dim entry), on latent pools filled through
the paged append: mixed lengths, ragged last tiles, empty sequences, head
counts that are not multiples of 16, forced single and many token splits,
and the restart taken when a later score exceeds the running max by more
than the kernel's headroom."""

import numpy as np
import pytest
import torch

import oracle as O
import vkv
from gpu_util import attn_tol, dev, values

pytestmark = pytest.mark.gpu

DK, DV, BS = 576, 512, 64


class Latent:
    """Latent pool with per-sequence random (permuted) block tables."""

    def __init__(self, rng, lens, nblocks=None, entries=None):
        self.lens = list(lens)
        need = sum((L + BS - 1) // BS for L in self.lens)
        nblocks = nblocks or need + 4
        self.pool = vkv.PagedPool(nblocks, BS, 1, 1, DK, dtype=vkv.BF16, bits=8, group_size=64,
                                  v_head_dim=DV, flags=vkv.VIEW_KEYS_ONLY)
        free = list(rng.permutation(np.arange(1, nblocks)))
        self.tables = [[int(free.pop()) for _ in range((L + BS - 1) // BS)] for L in self.lens]
        if entries is None:
            entries = [O.from_f32((rng.standard_normal((L, DK)) * 0.5).astype(np.float32), O.BF16)
                       for L in self.lens]
        self.entries = entries
        slots = [self.tables[s][p // BS] * BS + p % BS for s, L in enumerate(self.lens)
                 for p in range(L)]
        if slots:
            x = np.concatenate([e.reshape(-1, 1, DK) for e in entries])
            self.pool.append(0, dev(x, O.BF16), None,
                             torch.tensor(slots, dtype=torch.int32, device="cuda"))
        width = max(1, max(len(t) for t in self.tables))
        tab = np.zeros((len(self.lens), width), np.int32)
        for s, t in enumerate(self.tables):
            tab[s, :len(t)] = t
        self.tab = torch.from_numpy(tab).cuda()
        self.len_dev = torch.tensor(self.lens, dtype=torch.int32, device="cuda")

    def view(self, with_lens=True):
        return self.pool.view(0, self.tab, self.len_dev if with_lens else None, max(self.lens))

    def oracle(self, q, scale):
        """q: bf16 bits [B, H, 576] -> fp64 [B, H, 512]."""
        T = max(1, max(self.lens))
        x = np.zeros((len(self.lens), T, DK), np.uint16)
        for s, e in enumerate(self.entries):
            x[s, :len(e)] = e
        cq, cs, cb, _ = O.quantize(x, O.BF16, 64, 8)
        return O.mla_decode(O.to_f32(q, O.BF16), cq, O.to_f32(cs, O.BF16), O.to_f32(cb, O.BF16),
                            np.array(self.lens, np.int32), scale, Dv=DV, group=64, bits=8)


def run(L, q, scale, splits=None, with_lens=True):
    old = vkv.get_option("mla_splits")
    try:
        if splits is not None:
            vkv.set_option("mla_splits", splits)
        out = vkv.mla_decode(dev(q, O.BF16), L.view(with_lens), scale)
        torch.cuda.synchronize()
    finally:
        vkv.set_option("mla_splits", old)
    return values(out, O.BF16)


def check(got, ref, lens):
    for s, L in enumerate(lens):
        if L == 0:
            assert np.all(got[s] == 0), s
        else:
            bad = np.abs(got[s] - ref[s]) > attn_tol(O.BF16, ref[s])
            assert not bad.any(), (s, np.abs(got[s] - ref[s]).max())


@pytest.mark.parametrize("H", [128, 16, 20, 192])
@pytest.mark.parametrize("splits", [None, 1, 3])
def test_mla_matches_oracle(H, splits):
    rng = np.random.default_rng(1000 + H + 7 * (splits or 0))
    lens = [300, 1, 129, 64, 0]
    L = Latent(rng, lens)
    q = O.from_f32(rng.standard_normal((len(lens), H, DK)).astype(np.float32), O.BF16)
    scale = 192 ** -0.5
    got = run(L, q, scale, splits)
    check(got, L.oracle(q, scale), lens)


def test_mla_long_sequences_default_split():
    rng = np.random.default_rng(77)
    lens = [4096, 2500, 33]
    L = Latent(rng, lens)
    q = O.from_f32(rng.standard_normal((len(lens), 128, DK)).astype(np.float32), O.BF16)
    scale = 192 ** -0.5
    check(run(L, q, scale), L.oracle(q, scale), lens)


def test_mla_without_seq_lens():
    rng = np.random.default_rng(5)
    lens = [200, 200]
    L = Latent(rng, lens)
    q = O.from_f32(rng.standard_normal((2, 128, DK)).astype(np.float32), O.BF16)
    scale = 0.07
    check(run(L, q, scale, with_lens=False), L.oracle(q, scale), lens)


@pytest.mark.parametrize("splits", [1, 2])
def test_mla_restart_on_late_large_score(splits):
    """The first tile's scores are near zero and a later token scores far
    above them (more than 64 in log2 units), so the kernel must redo its
    split with the larger running max."""
    rng = np.random.default_rng(9)
    lens = [160, 97]
    ent = []
    for n in lens:
        x = rng.standard_normal((n, DK)).astype(np.float32) * 0.05
        x[:, 0] = 0.0
        x[100 % n, 0] = 8.0
        x[70, 0] = 6.0
        ent.append(O.from_f32(x, O.BF16))
    L = Latent(rng, lens, entries=ent)
    q = np.zeros((2, 64, DK), np.float32)
    q[:, :, 0] = 30.0
    q[:, :, 1:] = rng.standard_normal((2, 64, DK - 1)) * 0.1
    q = O.from_f32(q, O.BF16)
    scale = 1.0
    ref = L.oracle(q, scale)
    check(run(L, q, scale, splits), ref, lens)


def test_mla_rejects_non_latent_view():
    pool = vkv.PagedPool(8, 32, 1, 2, 128, dtype=vkv.BF16, bits=8)
    tab = torch.zeros((1, 2), dtype=torch.int32, device="cuda")
    view = pool.view(0, tab, None, 32)
    with pytest.raises(RuntimeError, match="keys-only"):
        vkv.mla_decode(torch.zeros((1, 4, 128), dtype=torch.bfloat16, device="cuda"), view, 0.1)
