"""Test infrastructure only: a numpy restatement of MLX's seeded random streams.

This module is part of the CPU oracle.  Only tests, the smoke check and the
CPU-baseline leg of the benchmark may use it; the product never does.

Why it exists: the reference's own seeded known-answer tests
(`Tests/MLXTests/IntegrationTests.swift:22-29` `testRandomSeed`,
`:3890-3923` `testQuantize`, `Tests/MLXTests/MLXFastKernelTests.swift:101-111`
`testFastSDPAOutput`) only become usable golden vectors if the inputs they
draw from `MLXRandom` can be reproduced.  MLX's core is not vendored in the
reference (`Source/Cmlx/mlx` is an empty submodule, `.gitmodules:1-3`), so
the algorithm is restated from its published description:

* Threefry-2x32 with 20 rounds (Salmon, Moraes, Dror, Shaw, "Parallel random
  numbers: as easy as 1, 2, 3", SC'11; Random123 rotation constants
  R = {13,15,26,6}, {17,29,16,24}, key-schedule parity 0x1BD11BDA) -- the
  counter-based generator behind MLX's `random::bits` (MLX core, fork pin
  a828cb4726f603d1cc9ac63359cd563865fdf8f6 per
  `docs/GEMMA4_QAT_CACHE_CORRECTNESS_CHECKPOINT_2026-07-19.md:292`).
* MLX conventions on top of it: `key(seed) = [seed >> 32, seed & 0xffffffff]`;
  `bits` fills the first and second half of each key's output from the two
  words of one Threefry call on counter pair (i, half + i); the global key
  sequence splits the current key into two rows and keeps the first;
  `uniform` divides the raw 32-bit words (converted to float32) by 2**32 and
  clamps below 1; `normal` maps uniform(-1+ulp, 1) through sqrt(2)*erfinv.

The restatement is pinned against the reference tests' numbers in
`tests/test_oracle_golden.py` (scalar normal for seed 864, the [4,3] means of
`testAddOp`), which fixes every convention listed above.
"""
from __future__ import annotations

import numpy as np

_ROT = ((13, 15, 26, 6), (17, 29, 16, 24))
_M32 = 0xFFFFFFFF


def _rotl(x: np.ndarray, r: int) -> np.ndarray:
    return ((x << np.uint32(r)) | (x >> np.uint32(32 - r))) & np.uint32(_M32)


def threefry2x32(key: tuple[int, int], c0: np.ndarray, c1: np.ndarray):
    """Threefry-2x32-20 of counter pairs (c0, c1) under `key` (vectorised)."""
    k0, k1 = np.uint32(key[0]), np.uint32(key[1])
    ks = (k0, k1, np.uint32((int(k0) ^ int(k1) ^ 0x1BD11BDA) & _M32))
    with np.errstate(over="ignore"):
        x0 = (c0.astype(np.uint32) + ks[0]).astype(np.uint32)
        x1 = (c1.astype(np.uint32) + ks[1]).astype(np.uint32)
        for i in range(5):
            for r in _ROT[i % 2]:
                x0 = (x0 + x1).astype(np.uint32)
                x1 = _rotl(x1, r)
                x1 = x1 ^ x0
            x0 = (x0 + ks[(i + 1) % 3]).astype(np.uint32)
            x1 = (x1 + ks[(i + 2) % 3] + np.uint32(i + 1)).astype(np.uint32)
    return x0, x1


def key(seed: int) -> tuple[int, int]:
    return ((seed >> 32) & _M32, seed & _M32)


def bits(key_: tuple[int, int], n_words: int) -> np.ndarray:
    """`n_words` 32-bit words drawn from one key (the 4-byte-width case)."""
    half = n_words // 2
    odd = n_words % 2
    out = np.empty(n_words, dtype=np.uint32)
    if half:
        i = np.arange(half, dtype=np.uint64)
        a, b = threefry2x32(key_, i, i + half + odd)
        out[:half] = a
        out[half + odd:] = b
    if odd:
        a, _ = threefry2x32(key_, np.array([half], np.uint64), np.array([0], np.uint64))
        out[half] = a[0]
    return out


def split(key_: tuple[int, int]):
    w = bits(key_, 4).reshape(2, 2)
    return (int(w[0, 0]), int(w[0, 1])), (int(w[1, 0]), int(w[1, 1]))


class KeySequence:
    """The process-global key stream that `MLXRandom.seed(s)` resets."""

    def __init__(self, seed: int):
        self.key = key(seed)

    def next(self):
        self.key, sub = split(self.key)
        return sub


def uniform_from_key(key_: tuple[int, int], shape, low: float = 0.0,
                     high: float = 1.0) -> np.ndarray:
    """`uniform` drawing from an explicit key (MLXRandom.uniform(key:))."""
    n = int(np.prod(shape)) if len(shape) else 1
    w = bits(key_, n)
    lo = np.float32(low)
    rng = np.float32(np.float32(high) - lo)
    u = w.astype(np.float32) / np.float32(4294967296.0)
    u = np.minimum(u, np.nextafter(np.float32(1.0), np.float32(0.0)))
    return (rng * u + lo).astype(np.float32).reshape(shape)


def uniform(seq: KeySequence, shape, low: float = 0.0, high: float = 1.0) -> np.ndarray:
    return uniform_from_key(seq.next(), shape, low, high)


def normal(seq: KeySequence, shape) -> np.ndarray:
    from scipy.special import erfinv

    lo = float(np.nextafter(np.float32(-1.0), np.float32(0.0)))
    u = uniform(seq, shape, lo, 1.0)
    return (np.float32(np.sqrt(2.0)) * erfinv(u.astype(np.float64)).astype(np.float32)).astype(
        np.float32
    )


def normal_uniforms(key_: tuple[int, int], shape) -> np.ndarray:
    """The uniform(-1 + ulp, 1) draws MLXRandom.normal(key:) maps through
    sqrt(2) * erfinv."""
    lo = float(np.nextafter(np.float32(-1.0), np.float32(0.0)))
    return uniform_from_key(key_, shape, lo, 1.0)
