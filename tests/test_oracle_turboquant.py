"""Pins for the TurboQuant restatement (oracle/tq_oracle.c, oracle.tq_*),
each against something other than the restated formula:

  * the Lloyd-Max codebook (TQCodebook.swift:103-160) against scipy
    quadrature of the sphere-coordinate density (1 - x^2)^((d-3)/2), a Monte
    Carlo estimate of the cell means from points drawn on the sphere, and the
    Gaussian Lloyd-Max levels (J. Max, 1960) that the density tends to;
  * the rotation signs (TQHadamard.swift:52-62) against the POSIX drand48
    linear congruential generator written out here;
  * MLX's f32 erfinv (erf.h:43-76) against scipy.special.erfinv, and the
    seeded normals it produces against the reference's known answers;
  * the Hadamard rotation (TQHadamard.swift:85-153) against
    scipy.linalg.hadamard, blockwise for dimensions that are not powers of 2;
  * the encoder / decoder (TQEncoder.swift:135-345): distortion equal to the
    codebook's own expected distortion, the QJL correction's unbiased inner
    products (the property the reference cites it for, TQQJL.swift:8-37),
    sign bits against a double-precision projection, norms against double
    arithmetic, bit packing against per-element bit extraction, and the
    sink / tail / dtype promotion rules."""
import numpy as np
import pytest
from scipy import integrate, linalg, special

import mlx_random as mr
import oracle as O


def _density(d):
    c = np.exp(special.gammaln(d / 2) - 0.5 * np.log(np.pi) - special.gammaln((d - 1) / 2))
    return lambda x: c * (1 - x * x) ** ((d - 3) / 2)


@pytest.mark.parametrize("d,bits", [(128, 1), (128, 2), (128, 3), (128, 4), (64, 3), (16, 2)])
def test_codebook_is_the_lloyd_max_fixed_point(d, bits):
    cb = O.tq_codebook(d, bits).astype(np.float64)
    n = len(cb)
    assert np.all(np.diff(cb) > 0) and np.allclose(cb, -cb[::-1], atol=2e-6)
    f = _density(d)
    edges = np.concatenate([[-1.0], (cb[:-1] + cb[1:]) / 2, [1.0]])
    for i in range(n):
        mass = integrate.quad(f, edges[i], edges[i + 1], limit=200)[0]
        mom = integrate.quad(lambda x: x * f(x), edges[i], edges[i + 1], limit=200)[0]
        # a 10000-point grid: centroid error well below 1e-3 of the support
        assert abs(mom / mass - cb[i]) < 1e-3 / np.sqrt(d) * 3, (i, mom / mass, cb[i])


def test_codebook_cells_match_sphere_samples():
    rng = np.random.default_rng(0)
    d = 128
    g = rng.standard_normal((400000, 8))  # the first coordinates of sphere points
    rest = rng.chisquare(d - 8, 400000)
    x = g[:, 0] / np.sqrt((g * g).sum(1) + rest)
    cb = O.tq_codebook(d, 3).astype(np.float64)
    cell = np.searchsorted((cb[:-1] + cb[1:]) / 2, x)
    for i in range(len(cb)):
        xs = x[cell == i]
        se = xs.std() / np.sqrt(len(xs))
        assert abs(xs.mean() - cb[i]) < 5 * se + 1e-5, (i, xs.mean(), cb[i])


def test_codebook_tends_to_gaussian_lloyd_max():
    # Max (1960), unit-variance Gaussian optimum levels
    # (the 10000-point grid of [-1, 1] resolves the +-3/sqrt(d) support
    # less finely as d grows, so the limit is checked at a moderate d)
    levels = {1: [0.7979], 2: [0.4528, 1.5104], 3: [0.2451, 0.7560, 1.3440, 2.1520]}
    d = 256
    for bits, pos in levels.items():
        cb = O.tq_codebook(d, bits) * np.sqrt(d)
        assert np.allclose(cb[len(cb) // 2:], pos, rtol=1.5e-2), (bits, cb)


def _drand48(seed, n):
    x = ((seed & 0xFFFFFFFF) << 16) | 0x330E
    out = []
    for _ in range(n):
        x = (0x5DEECE66D * x + 0xB) & ((1 << 48) - 1)
        out.append(x / 2.0 ** 48)
    return np.array(out)


@pytest.mark.parametrize("seed", [42, 0, 7, 1042])
def test_signs_follow_posix_drand48(seed):
    got = O.tq_random_signs(200, seed)
    want = np.where(_drand48(seed, 200) < 0.5, -1.0, 1.0)
    assert np.array_equal(got, want)


def _ulps(a, b):
    a, b = np.float32(a), np.float32(b)
    ia = np.array([a], np.float32).view(np.int32)[0]
    ib = np.array([b], np.float32).view(np.int32)[0]
    return abs(int(ia) - int(ib))


def test_erfinv_matches_scipy():
    xs = np.concatenate([np.linspace(-0.999999, 0.999999, 4001), [0.0, 1e-30, -1e-7, 0.5, 0.9999]])
    xs = xs.astype(np.float32)
    got = O.tq_erfinv(xs)
    want = special.erfinv(xs.astype(np.float64)).astype(np.float32)
    worst = max(_ulps(g, w) for g, w in zip(got, want))
    assert worst <= 3, worst


def test_qjl_matrix_and_seeded_normals(golden):
    # the reference's known seeded normals, drawn through the f32 erfinv
    g = golden["random_seed_normal"]
    seq = mr.KeySequence(g["seed"])
    u = mr.uniform(seq, (), float(np.nextafter(np.float32(-1), np.float32(0))), 1.0)
    v = np.float32(np.sqrt(2.0)) * O.tq_erfinv(np.array([u]))[0]
    assert abs(v - g["value"]) < g["accuracy"]
    S = O.tq_qjl_matrix(128, 1042)
    ref = mr.normal_uniforms(mr.key(1042), (128, 128))
    ref = (np.float32(np.sqrt(2.0)) * special.erfinv(ref.astype(np.float64))).astype(np.float32)
    d = np.abs(S - ref) / np.maximum(np.abs(ref), 1e-6)
    assert d.max() < 4 * 2.0 ** -23
    assert abs(S.mean()) < 0.02 and abs(S.std() - 1) < 0.02


@pytest.mark.parametrize("dim", [2, 8, 64, 128, 256])
def test_hadamard_is_scipy_sylvester(dim):
    rng = np.random.default_rng(dim)
    x = rng.standard_normal((5, dim)).astype(np.float32)
    s = O.tq_random_signs(dim, 42)
    H = linalg.hadamard(dim) / np.sqrt(dim)
    y = O.tq_hadamard(x, s)
    assert np.allclose(y, (x * s) @ H.T, atol=1e-5)
    back = O.tq_hadamard(y, s, inverse=True)
    assert np.allclose(back, x, atol=1e-5)


@pytest.mark.parametrize("dim,blocks", [(192, [128, 64]), (80, [64, 16]), (576, [512, 64]),
                                        (100, [64, 32, 4])])
def test_hadamard_blocks_for_other_dims(dim, blocks):
    import ctypes as C
    out = (C.c_int * 32)()
    n = O.lib().tqo_pow2_blocks(dim, out)
    assert list(out[:n]) == blocks
    rng = np.random.default_rng(dim)
    x = rng.standard_normal((3, dim)).astype(np.float32)
    s = O.tq_random_signs(dim, 42)
    y = O.tq_hadamard(x, s)
    off = 0
    for b in blocks:
        H = linalg.hadamard(b) / np.sqrt(b)
        assert np.allclose(y[:, off:off + b], (x[:, off:off + b] * s[off:off + b]) @ H.T, atol=1e-5)
        off += b


@pytest.mark.parametrize("bits", [1, 2, 3, 4, 5, 6, 8])
def test_bit_packing_layout(bits):
    rng = np.random.default_rng(bits)
    n = 1000
    v = rng.integers(0, 1 << bits, n).astype(np.uint8)
    p = O.tq_pack_bits(v, bits)
    vpw = 32 // bits
    assert p.size == -(-n // vpw)
    for e in range(n):
        assert (int(p[e // vpw]) >> ((e % vpw) * bits)) & ((1 << bits) - 1) == v[e]
    assert np.array_equal(O.tq_unpack_bits(p, bits, n), v)


def _expected_distortion(d, cb):
    f = _density(d)
    edges = np.concatenate([[-1.0], (cb[:-1] + cb[1:]) / 2, [1.0]])
    return sum(integrate.quad(lambda x: (x - c) ** 2 * f(x), lo, hi, limit=200)[0]
               for c, lo, hi in zip(cb, edges[:-1], edges[1:]))


def test_value_distortion_is_the_codebook_distortion():
    st = O.TQState(128, 3, 3)
    rng = np.random.default_rng(5)
    x = rng.standard_normal((1, 4, 600, 128)).astype(np.float32)
    enc = O.tq_encode(x, O.F32, st, keys=False, sink=0, tail=0)
    dec, dt = O.tq_decode(enc, st, keys=False)
    assert dt == O.F16 and dec.shape == x.shape
    # the error per unit-norm vector, in the rotated domain, is the scalar
    # quantizer's: d * E[(X - Q(X))^2] summed over the coordinates
    nrm = np.linalg.norm(x, axis=-1, keepdims=True)
    err = (((dec - x) / nrm) ** 2).sum(-1).mean()
    want = 128 * _expected_distortion(128, st.value_codebook.astype(np.float64))
    assert abs(err - want) / want < 0.05, (err, want)


def test_qjl_makes_inner_products_unbiased():
    st = O.TQState(128, 3, 3)
    rng = np.random.default_rng(6)
    k = rng.standard_normal((1, 8, 500, 128)).astype(np.float32)
    q = rng.standard_normal((8, 128)).astype(np.float32)
    enc = O.tq_encode(k, O.F32, st, keys=True, sink=0, tail=0)
    dec, _ = O.tq_decode(enc, st, keys=True)
    # the same codes without the QJL term: codebook levels only
    mse = enc.copy()
    mse["res_norms"] = O.from_f32(np.zeros(4000, np.float32), O.F16)
    dmse, _ = O.tq_decode(mse, st, keys=True)
    true = np.einsum("hd,htd->ht", q, k[0]).astype(np.float64)
    e_qjl = np.einsum("hd,htd->ht", q, dec[0]) - true
    e_mse = np.einsum("hd,htd->ht", q, dmse[0]) - true
    # a Lloyd-Max quantizer shrinks projections: E[X Q(X)] = E[Q(X)^2] =
    # (1 - D) E[X^2], so the MSE-only estimate regresses on <q, k> with
    # slope -D (about -0.12 at 2 bits); QJL removes that bias
    slope = lambda e: (e * true).sum() / (true * true).sum()
    D = 128 * _expected_distortion(128, st.key_codebook.astype(np.float64))
    assert abs(slope(e_mse) + D) < 0.02, (slope(e_mse), D)
    assert abs(slope(e_qjl)) < 0.02, slope(e_qjl)
    assert abs(e_qjl.mean()) < 5 * e_qjl.std() / np.sqrt(e_qjl.size)


def test_encoder_fields_against_double_arithmetic():
    st = O.TQState(128, 3, 3)
    rng = np.random.default_rng(7)
    for dtype in (O.F32, O.F16, O.BF16):
        x = O.to_f32(O.from_f32(rng.standard_normal((2, 2, 30, 128)).astype(np.float32) * 3, dtype),
                     dtype)
        enc = O.tq_encode(x, dtype, st, keys=True, sink=2, tail=3)
        mid = x[:, :, 2:27].reshape(-1, 128).astype(np.float64)
        nrm = np.sqrt((mid * mid).sum(1))
        vn = O.to_f32(enc["vec_norms"].reshape(-1), O.F16)
        ulp = {O.F32: 2.0 ** -23, O.F16: 2.0 ** -10, O.BF16: 2.0 ** -7}[dtype]
        assert np.all(np.abs(vn - nrm) <= (2 * ulp + 2.0 ** -11) * nrm), dtype
        # rotated unit vectors: the unit vector in T, signs, H / sqrt(d)
        H = linalg.hadamard(128) / np.sqrt(128)
        unit = mid / nrm[:, None]
        assert np.allclose(enc["rot"], (unit * st.signs) @ H.T, atol=4 * ulp)
        # codes: the cell of each rotated value; signs of a double projection
        bnd = (st.key_codebook[:-1] + st.key_codebook[1:]) / 2
        assert np.array_equal(enc["idx"], np.searchsorted(bnd, enc["rot"], side="left")
                              .astype(np.uint8))
        r = enc["rot"].astype(np.float64) - st.key_codebook[enc["idx"]]
        p64 = r @ st.S.astype(np.float64).T
        bound = 128 * 2.0 ** -24 * (np.abs(r) @ np.abs(st.S.astype(np.float64)).T)
        sure = np.abs(p64) > bound
        assert np.array_equal(enc["sgn"][sure], (p64 >= 0)[sure]) and sure.mean() > 0.999
        rn = O.to_f32(enc["res_norms"].reshape(-1), O.F16)
        assert np.allclose(rn, np.sqrt((r * r).sum(1)), rtol=2.0 ** -10, atol=1e-7)
        # the packed fields hold exactly these codes and signs
        n = enc["idx"].size
        assert np.array_equal(O.tq_unpack_bits(enc["indices"], 2, n), enc["idx"].reshape(-1))
        assert np.array_equal(O.tq_unpack_bits(enc["qjl"], 1, n), enc["sgn"].reshape(-1))


def test_sink_tail_and_promotion():
    st = O.TQState(64, 4, 4)
    rng = np.random.default_rng(8)
    for dtype, sink, tail, want in [(O.F16, 4, 8, O.F16), (O.BF16, 4, 8, O.F32),
                                    (O.F32, 4, 0, O.F32), (O.BF16, 0, 0, O.F16),
                                    (O.BF16, 0, 5, O.F32)]:
        x = O.to_f32(O.from_f32(rng.standard_normal((1, 2, 40, 64)).astype(np.float32), dtype),
                     dtype)
        for keys in (True, False):
            enc = O.tq_encode(x, dtype, st, keys=keys, sink=sink, tail=tail)
            assert enc["shape"] == [1, 2, 40 - sink - tail, 64]
            dec, dt = O.tq_decode(enc, st, keys=keys)
            assert dt == want and dec.shape == x.shape
            assert np.array_equal(dec[:, :, :sink], x[:, :, :sink])
            assert np.array_equal(dec[:, :, 40 - tail:], x[:, :, 40 - tail:])
            mid = dec[:, :, sink:40 - tail]
            assert np.array_equal(mid, O.to_f32(O.from_f32(mid, O.F16), O.F16))
    with pytest.raises(AssertionError):
        O.tq_encode(np.zeros((1, 1, 6, 64), np.float32), O.F32, st, True, sink=4, tail=2)


def test_power_of_two_scaling_leaves_the_codes():
    """Scaling a vector by 2^k scales its norm by exactly 2^k and leaves the
    unit vector, hence every code and sign, unchanged; the decoded vector
    scales with the stored norm."""
    st = O.TQState(128, 3, 3)
    rng = np.random.default_rng(9)
    x = rng.standard_normal((1, 2, 20, 128)).astype(np.float32)
    for keys in (True, False):
        a = O.tq_encode(x, O.F32, st, keys=keys, sink=0, tail=0)
        b = O.tq_encode(x * np.float32(8), O.F32, st, keys=keys, sink=0, tail=0)
        assert np.array_equal(a["idx"], b["idx"])
        va, vb = (O.to_f32(e["vec_norms"].reshape(-1), O.F16) for e in (a, b))
        assert np.array_equal(va * 8, vb)
        if keys:
            assert np.array_equal(a["sgn"], b["sgn"])
            assert np.array_equal(a["res_norms"], b["res_norms"])
        da, _ = O.tq_decode(a, st, keys=keys)
        db, _ = O.tq_decode(b, st, keys=keys)
        normal = np.abs(da) >= 2.0 ** -14  # f16 subnormals round on a fixed grid
        assert np.array_equal((da * 8)[normal], db[normal]) and normal.mean() > 0.99
