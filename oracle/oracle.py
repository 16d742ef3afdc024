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
        [vp, i32] + [vp] * 6 + [i32] * 8 + [f32, i32, vp, vp] + [i64] * 4 + [i32, vp, vp]
    )
    L.vkvo_mla_decode.argtypes = [vp, vp, vp, vp, i32, i32, i32, vp, i32, i32, i32, i32, f32, vp]
    L.vkvo_quantized_decode_batch.argtypes = (
        [vp, i32] + [vp] * 6 + [i32, vp, vp, i32, i32, i32, i32, i32, f32, i32, i32, vp]
    )


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
                   rounding=QMV, bound=False):
    """Reference-layout quantized cache; scales/biases as f32 values.

    rounding: EXACT, QMV (default: the reference's decode arithmetic), QMM
    or QMV_ACC_T (see vkvo_quantized_sdpa).  With bound=True also returns
    the per-output weight-rounding bound sum_t |w_t - p_t| |v_t|."""
    q = np.ascontiguousarray(q, dtype=np.float32)
    B, Hq, L, D = q.shape
    Hkv, T = kq.shape[1], kq.shape[2]
    arrs = [np.ascontiguousarray(x, dtype=t) for x, t in
            ((kq, np.uint32), (ks, np.float32), (kb, np.float32),
             (vq, np.uint32), (vs, np.float32), (vb, np.float32))]
    mode, mb, mf, st, keep = _mask_args(mask, B, Hq, L, T)
    out = np.empty((B, Hq, L, D), np.float64)
    wb = np.empty((B, Hq, L, D), np.float64) if bound else None
    lib().vkvo_quantized_sdpa(_p(q), q_dtype, *[_p(a) for a in arrs], B, Hq, Hkv, L, T, D,
                              group, bits, scale, mode, _p(mb), _p(mf), *st, rounding,
                              _p(out), _p(wb))
    return (out, wb) if bound else out


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
