"""Test infrastructure only: ctypes front end of the C oracle (liboracle.so).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this module.  Arrays are numpy; dtype codes follow the product ABI
(0 = f32, 1 = f16, 2 = bf16).  bf16 arrays are carried as uint16 bit patterns.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

F32, F16, BF16 = 0, 1, 2

# quantized-SDPA arithmetic (vkvo_quantized_sdpa): exact fp64; scores and
# weights rounded to the query dtype with an fp32 softmax on the vector (qmv)
# and matrix (qmm) paths; the same with the softmax computed in the query
# dtype (softmax(precise: false), the reference's arithmetic) on each path.
EXACT, QMV, QMM, QMV_ACC_T, QMM_ACC_T = 0, 1, 2, 3, 4
# the reference's decode (one query token) and multi-token arithmetic
REF_DECODE, REF_CHUNK = QMV_ACC_T, QMM_ACC_T

_lib = None


def build() -> None:
    subprocess.run(["make", "-s", "-C", HERE, "-B", "liboracle.so"], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        _lib = C.CDLL(LIB_PATH)
        _declare(_lib)
    return _lib


def _p(a):
    return a.ctypes.data_as(C.c_void_p) if a is not None else None


def _declare(L):
    vp, i64, i32, f32 = C.c_void_p, C.c_int64, C.c_int, C.c_float
    L.vkvo_f32_to_bf16.restype = C.c_uint16
    L.vkvo_f32_to_bf16.argtypes = [f32]
    L.vkvo_bf16_to_f32.restype = f32
    L.vkvo_bf16_to_f32.argtypes = [C.c_uint16]
    L.vkvo_f32_to_f16.restype = C.c_uint16
    L.vkvo_f32_to_f16.argtypes = [f32]
    L.vkvo_f16_to_f32.restype = f32
    L.vkvo_f16_to_f32.argtypes = [C.c_uint16]
    L.vkvo_to_f32.argtypes = [vp, i32, i64, vp]
    L.vkvo_from_f32.argtypes = [vp, i64, i32, vp]
    L.vkvo_quantize.restype = i64
    L.vkvo_quantize.argtypes = [vp, i32, i64, i32, i32, i32, vp, vp, vp]
    L.vkvo_dequantize.argtypes = [vp, vp, vp, i32, i64, i32, i32, i32, i32, vp]
    L.vkvo_dequantize_rule_split.restype = i64
    L.vkvo_dequantize_rule_split.argtypes = [vp, vp, vp, i32, i64, i32, i32, i32]
    L.vkvo_sdpa.argtypes = [vp, vp, vp] + [i32] * 7 + [f32, i32, vp, vp] + [i64] * 4 + [i32, vp, vp]
    L.vkvo_quantized_sdpa.argtypes = (
        [vp, i32] + [vp] * 6 + [i32] * 8 + [f32, i32, vp, vp] + [i64] * 4 + [i32, vp, vp, vp]
    )
    L.vkvo_mla_decode.argtypes = [vp, vp, vp, vp, i32, i32, i32, vp, i32, i32, i32, i32, f32, vp]
    L.vkvo_quantized_decode_batch.argtypes = (
        [vp, i32] + [vp] * 6 + [i32, vp, vp, i32, i32, i32, i32, i32, f32, i32, i32, vp]
    )
    L.tqo_codebook.argtypes = [i32, i32, i32, vp]
    L.tqo_random_signs.argtypes = [i32, C.c_long, vp]
    L.tqo_erfinv.restype = f32
    L.tqo_erfinv.argtypes = [f32]
    L.tqo_normal_from_uniform.argtypes = [vp, i64, vp]
    L.tqo_hadamard.argtypes = [vp, i64, i32, vp, i32]
    L.tqo_pow2_blocks.restype = i32
    L.tqo_pow2_blocks.argtypes = [i32, vp]
    L.tqo_encode.argtypes = [vp, i32, i64, i32, vp, vp, i32] + [vp] * 7
    L.tqo_decode.argtypes = [vp, vp, vp, vp, i64, i32, vp, vp, vp, vp]


def np_dtype(code):
    return {F32: np.float32, F16: np.uint16, BF16: np.uint16}[code]


def to_f32(a: np.ndarray, dtype: int) -> np.ndarray:
    a = np.ascontiguousarray(a)
    out = np.empty(a.shape, np.float32)
    lib().vkvo_to_f32(_p(a), dtype, a.size, _p(out))
    return out


def from_f32(a: np.ndarray, dtype: int) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.float32)
    out = np.empty(a.shape, np_dtype(dtype))
    lib().vkvo_from_f32(_p(a), a.size, dtype, _p(out))
    return out


def round_to(a: np.ndarray, dtype: int) -> np.ndarray:
    return to_f32(from_f32(a, dtype), dtype)


def quantize(w: np.ndarray, dtype: int, group: int = 64, bits: int = 4):
    """Returns (wq u32 [..., D*bits/32], scales [..., D/g], biases, ties)."""
    w = np.ascontiguousarray(w)
    D = w.shape[-1]
    rows = w.size // D
    wq = np.empty(w.shape[:-1] + (D * bits // 32,), np.uint32)
    sc = np.empty(w.shape[:-1] + (D // group,), np_dtype(dtype))
    bi = np.empty_like(sc)
    ties = lib().vkvo_quantize(_p(w), dtype, rows, D, group, bits, _p(wq), _p(sc), _p(bi))
    return wq, sc, bi, int(ties)


def dequantize(wq, scales, biases, dtype: int, group: int = 64, bits: int = 4, rule: int = 0):
    """rule 0: T(scale*q + bias) rounded once; rule 1: T(T(scale*q) + bias)."""
    wq = np.ascontiguousarray(wq, dtype=np.uint32)
    D = wq.shape[-1] * 32 // bits
    rows = wq.size // wq.shape[-1]
    out = np.empty(wq.shape[:-1] + (D,), np_dtype(dtype))
    lib().vkvo_dequantize(
        _p(wq), _p(np.ascontiguousarray(scales)), _p(np.ascontiguousarray(biases)),
        dtype, rows, D, group, bits, rule, _p(out)
    )
    return out


def dequantize_rule_split(wq, scales, biases, dtype: int, group: int = 64, bits: int = 4) -> int:
    """Elements where the one- and two-rounding dequantize rules differ."""
    wq = np.ascontiguousarray(wq, dtype=np.uint32)
    D = wq.shape[-1] * 32 // bits
    rows = wq.size // wq.shape[-1]
    return int(lib().vkvo_dequantize_rule_split(
        _p(wq), _p(np.ascontiguousarray(scales)), _p(np.ascontiguousarray(biases)),
        dtype, rows, D, group, bits))


def _mask_args(mask, B, H, L, T):
    """mask: None | 'causal' | bool array | float array broadcastable to [B,H,L,T]."""
    if mask is None:
        return 0, None, None, (0, 0, 0, 0), None
    if isinstance(mask, str):
        assert mask == "causal"
        return 1, None, None, (0, 0, 0, 0), None
    m = np.asarray(mask)
    while m.ndim < 4:
        m = m[None]
    m = np.broadcast_to(m, (B, H, L, T))
    st = tuple(s // m.itemsize for s in m.strides)
    if m.dtype == np.bool_:
        mb = np.ascontiguousarray(m).view(np.uint8)
        st = tuple(s // mb.itemsize for s in mb.strides)
        return 2, mb, None, st, mb
    mf = np.ascontiguousarray(m, dtype=np.float32)
    st = tuple(s // 4 for s in mf.strides)
    return 3, None, mf, st, mf


def sdpa(q, k, v, scale, mask=None, q_dtype=F32, sinks=None):
    """q [B,Hq,L,D], k [B,Hkv,T,D], v [B,Hkv,T,Dv] as f32 values -> f64 out.
    An additive mask is read in q_dtype (rounded to it, keys below its
    lowest finite value skipped); sinks: optional [Hq] logits (values of
    q_dtype)."""
    q, k, v = (np.ascontiguousarray(x, dtype=np.float32) for x in (q, k, v))
    B, Hq, L, D = q.shape
    Hkv, T, Dv = k.shape[1], k.shape[2], v.shape[3]
    mode, mb, mf, st, keep = _mask_args(mask, B, Hq, L, T)
    sk = None if sinks is None else np.ascontiguousarray(sinks, dtype=np.float32)
    out = np.empty((B, Hq, L, Dv), np.float64)
    lib().vkvo_sdpa(_p(q), _p(k), _p(v), B, Hq, Hkv, L, T, D, Dv, scale, mode, _p(mb),
                    _p(mf), *st, q_dtype, _p(sk), _p(out))
    return out


def quantized_sdpa(q, q_dtype, kq, ks, kb, vq, vs, vb, scale, group=64, bits=4, mask=None,
                   rounding=QMV, bound=False, flip=False):
    """Reference-layout quantized cache; scales/biases as f32 values.

    rounding: EXACT, QMV (default: the reference's decode arithmetic), QMM
    or QMV_ACC_T (see vkvo_quantized_sdpa).  With bound=True also returns
    the per-output rounding bound (the weight term sum_t |w_t - p_t| |v_t|
    plus the score-boundary term); with flip=True instead the
    score-boundary term alone."""
    q = np.ascontiguousarray(q, dtype=np.float32)
    B, Hq, L, D = q.shape
    Hkv, T = kq.shape[1], kq.shape[2]
    arrs = [np.ascontiguousarray(x, dtype=t) for x, t in
            ((kq, np.uint32), (ks, np.float32), (kb, np.float32),
             (vq, np.uint32), (vs, np.float32), (vb, np.float32))]
    mode, mb, mf, st, keep = _mask_args(mask, B, Hq, L, T)
    out = np.empty((B, Hq, L, D), np.float64)
    wb = np.empty((B, Hq, L, D), np.float64) if bound else None
    fb = np.empty((B, Hq, L, D), np.float64) if flip else None
    lib().vkvo_quantized_sdpa(_p(q), q_dtype, *[_p(a) for a in arrs], B, Hq, Hkv, L, T, D,
                              group, bits, scale, mode, _p(mb), _p(mf), *st, rounding,
                              _p(out), _p(wb), _p(fb))
    if bound and flip:
        return out, wb, fb
    return (out, wb) if bound else (out, fb) if flip else out


def mla_decode(q, cq, cs, cb, lens, scale, Dv=512, group=64, bits=8):
    q = np.ascontiguousarray(q, dtype=np.float32)
    B, H, Dk = q.shape
    T = cq.shape[1]
    lens = np.ascontiguousarray(lens, dtype=np.int32)
    out = np.empty((B, H, Dv), np.float64)
    lib().vkvo_mla_decode(_p(q), _p(np.ascontiguousarray(cq, dtype=np.uint32)),
                          _p(np.ascontiguousarray(cs, dtype=np.float32)),
                          _p(np.ascontiguousarray(cb, dtype=np.float32)),
                          B, H, T, _p(lens), Dk, Dv, group, bits, scale, _p(out))
    return out


def quantized_decode_batch(q, q_dtype, kq, ks, kb, vq, vs, vb, lens, tok_off, Hkv, scale,
                           group=64, bits=4, threads=1, rounding=QMV):
    q = np.ascontiguousarray(q, dtype=np.float32)
    nseq, Hq, D = q.shape
    out = np.empty((nseq, Hq, D), np.float64)
    arrs = [np.ascontiguousarray(x) for x in (kq, ks, kb, vq, vs, vb)]
    lib().vkvo_quantized_decode_batch(
        _p(q), q_dtype, *[_p(a) for a in arrs], nseq,
        _p(np.ascontiguousarray(lens, dtype=np.int32)),
        _p(np.ascontiguousarray(tok_off, dtype=np.int64)), Hq, Hkv, D, group, bits, scale,
        rounding, threads, _p(out))
    return out


# ---------------------------------------------------------------- TurboQuant
# TurboQuant KV codec (Libraries/MLXLMCommon/TurboQuant/): tq_oracle.c plus
# the bit packing of TQBitPack.swift and the encoded-record layout of
# TQEncodedData.swift.
def tq_codebook(dim: int, bits: int, iterations: int = 200) -> np.ndarray:
    """TQCodebook.computeCodebook (TQCodebook.swift:103-160)."""
    out = np.empty(1 << bits, np.float32)
    lib().tqo_codebook(dim, bits, iterations, _p(out))
    return out


def tq_random_signs(dim: int, seed: int) -> np.ndarray:
    """TQHadamard.generateRandomSigns (TQHadamard.swift:52-62)."""
    out = np.empty(dim, np.float32)
    lib().tqo_random_signs(dim, C.c_long(seed), _p(out))
    return out


def tq_erfinv(a) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.float32)
    out = np.empty_like(a)
    f = lib().tqo_erfinv
    flat_in, flat_out = a.reshape(-1), out.reshape(-1)
    for i in range(flat_in.size):
        flat_out[i] = f(float(flat_in[i]))
    return out


def tq_qjl_matrix(dim: int, seed: int) -> np.ndarray:
    """TQQJL.generateProjection (TQQJL.swift:55-58): MLXRandom.normal([dim,
    dim], key(seed)) -- MLX's uniform draws mapped through its f32 erfinv."""
    import mlx_random as mr

    u = mr.normal_uniforms(mr.key(seed), (dim, dim))
    out = np.empty_like(u)
    lib().tqo_normal_from_uniform(_p(u), u.size, _p(out))
    return out


def tq_hadamard(x, signs, inverse=False) -> np.ndarray:
    """hadamardRotate / hadamardInverse (TQHadamard.swift:117-153) on rows."""
    y = np.array(x, dtype=np.float32, order="C", copy=True)
    dim = y.shape[-1]
    lib().tqo_hadamard(_p(y), y.size // dim, dim, _p(np.ascontiguousarray(signs, np.float32)),
                       int(inverse))
    return y


def tq_pack_bits(values, bits: int) -> np.ndarray:
    """TQBitPack.packBits (TQBitPack.swift:47-65): flat, 32 // bits values
    per u32 little-end first, zero-padded."""
    vpw = 32 // bits
    flat = np.asarray(values, np.uint32).reshape(-1)
    pad = (vpw - flat.size % vpw) % vpw
    flat = np.concatenate([flat, np.zeros(pad, np.uint32)]).reshape(-1, vpw)
    out = np.zeros(flat.shape[0], np.uint32)
    for i in range(vpw):
        out |= flat[:, i] << np.uint32(i * bits)
    return out


def tq_unpack_bits(packed, bits: int, n: int) -> np.ndarray:
    """TQBitPack.unpackBits (TQBitPack.swift:77-88)."""
    vpw = 32 // bits
    p = np.asarray(packed, np.uint32)
    cols = [(p >> np.uint32(i * bits)) & np.uint32((1 << bits) - 1) for i in range(vpw)]
    return np.stack(cols, -1).reshape(-1)[:n].astype(np.uint8)


def tq_pack_signs(bits01) -> np.ndarray:
    """TQBitPack.packSigns (TQBitPack.swift:95-112): bit 1 for +1."""
    return tq_pack_bits(bits01, 1)


class TQState:
    """TQEncoder.EncoderState (TQEncoder.swift:88-107)."""

    def __init__(self, dim: int, key_bits: int = 3, value_bits: int = 3, seed: int = 42):
        self.dim, self.key_bits, self.value_bits, self.seed = dim, key_bits, value_bits, seed
        self.signs = tq_random_signs(dim, seed)
        self.key_index_bits = max(key_bits - 1, 1)
        self.key_codebook = tq_codebook(dim, self.key_index_bits)
        self.value_index_bits = value_bits
        self.value_codebook = tq_codebook(dim, value_bits)
        self.S = tq_qjl_matrix(dim, seed + 1000)


def _promote(a: int, b: int) -> int:
    """MLX's type promotion among f32 / f16 / bf16: f16 with bf16 is f32."""
    return a if a == b else F32


def tq_encode(x, dtype: int, state: TQState, keys: bool, sink: int = 4, tail: int = 0) -> dict:
    """TQEncoder.encodeKeys / encodeValues (TQEncoder.swift:135-206,
    :262-312).  x: [B, H, T, D] values of `dtype` as f32.  Returns the
    EncodedKeys / EncodedValues fields (norms as f16 bit patterns, sink /
    tail as `dtype` values) plus the unpacked codes, signs, projections and
    rotated vectors for the tests."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    B, H, T, D = x.shape
    pre = min(max(sink, 0), T)
    tl = min(max(tail, 0), max(0, T - pre))
    mid = x[:, :, pre:T - tl]
    assert mid.shape[2] > 0, "TurboQuant encode requires at least one compressible token"
    rows = B * H * mid.shape[2]
    flat = np.ascontiguousarray(mid).reshape(rows, D)
    cb = state.key_codebook if keys else state.value_codebook
    ib = state.key_index_bits if keys else state.value_index_bits
    idx = np.empty((rows, D), np.uint8)
    sgn = np.empty((rows, D), np.uint8)
    vn = np.empty(rows, np.float32)
    rn = np.empty(rows, np.float32)
    proj = np.empty((rows, D), np.float32)
    rot = np.empty((rows, D), np.float32)
    S = state.S if keys else None
    lib().tqo_encode(_p(flat), dtype, rows, D, _p(state.signs), _p(cb), ib,
                     _p(S) if keys else None, _p(idx), _p(sgn), _p(vn), _p(rn), _p(proj), _p(rot))
    ms = mid.shape
    enc = {
        "indices": tq_pack_bits(idx, ib), "vec_norms": from_f32(vn, F16).reshape(ms[:3] + (1,)),
        "shape": list(ms), "index_bits": ib, "seed": state.seed,
        "sink": x[:, :, :pre] if pre else None, "tail": x[:, :, T - tl:] if tl else None,
        "dtype": dtype, "idx": idx, "rot": rot,
    }
    if keys:
        enc.update(qjl=tq_pack_signs(sgn), res_norms=from_f32(rn, F16).reshape(ms[:3] + (1,)),
                   sgn=sgn, proj=proj)
    return enc


def tq_decode(enc: dict, state: TQState, keys: bool):
    """TQEncoder.decodeKeys / decodeValues (TQEncoder.swift:214-255,
    :315-345) with the sink / tail concatenation; returns (values as f32,
    result dtype code)."""
    B, H, Tc, D = enc["shape"]
    rows = B * H * Tc
    idx = tq_unpack_bits(enc["indices"], enc["index_bits"], rows * D)
    cb = state.key_codebook if keys else state.value_codebook
    vn = to_f32(np.ascontiguousarray(enc["vec_norms"]).reshape(-1), F16)
    out = np.empty((rows, D), np.float32)
    if keys:
        sg = tq_unpack_bits(enc["qjl"], 1, rows * D)
        rn = to_f32(np.ascontiguousarray(enc["res_norms"]).reshape(-1), F16)
        lib().tqo_decode(_p(idx), _p(sg), _p(vn), _p(rn), rows, D, _p(state.signs), _p(cb),
                         _p(state.S), _p(out))
    else:
        lib().tqo_decode(_p(idx), None, _p(vn), None, rows, D, _p(state.signs), _p(cb), None,
                         _p(out))
    dec = out.reshape(B, H, Tc, D)
    dt = F16
    parts = [dec]
    if enc["sink"] is not None:
        parts.insert(0, enc["sink"])
        dt = _promote(enc["dtype"], dt)
    if enc["tail"] is not None:
        parts.append(enc["tail"])
        dt = _promote(enc["dtype"], dt)
    return np.concatenate(parts, axis=2).astype(np.float32), dt

