"""Helpers shared by the GPU parity tests: numpy <-> torch-on-HIP moves that
keep bf16/f16 as exact bit patterns, seeded inputs, and tolerances."""
import numpy as np
import torch

import oracle as O
import vkv

TORCH = {O.F32: torch.float32, O.F16: torch.float16, O.BF16: torch.bfloat16}


def dev(a: np.ndarray, dtype: int):
    """numpy array (uint16 bit patterns for f16/bf16, float32 for f32) -> cuda tensor."""
    if dtype == O.F32:
        return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).cuda()
    t = torch.from_numpy(np.ascontiguousarray(a).view(np.int16))
    return t.view(TORCH[dtype]).cuda()


def host(t) -> np.ndarray:
    """cuda tensor -> numpy bits (uint16 for 16-bit floats, uint32 for int32 codes)."""
    t = t.detach().contiguous().cpu()
    if t.dtype in (torch.float16, torch.bfloat16):
        return t.view(torch.int16).numpy().view(np.uint16)
    if t.dtype == torch.int32:
        return t.numpy().view(np.uint32)
    return t.numpy()


def values(t, dtype: int) -> np.ndarray:
    """cuda tensor -> float32 values."""
    return O.to_f32(host(t), dtype) if dtype != O.F32 else host(t).astype(np.float32)


def rand_bits(rng, shape, dtype: int, std=1.0, outliers=0):
    x = (rng.standard_normal(shape) * std).astype(np.float32)
    if outliers:
        ch = rng.choice(shape[-1], outliers, replace=False)
        x[..., ch] *= 20.0
    return O.from_f32(x, dtype)


def attn_tol(dtype: int, ref: np.ndarray) -> np.ndarray:
    """Attention tolerance: 2e-2 max-abs for 16-bit outputs and 1e-4 for f32,
    plus one unit in the last place of the output dtype (the rounding of the
    stored result itself)."""
    ulp = {O.BF16: 2.0 ** -8, O.F16: 2.0 ** -11, O.F32: 2.0 ** -23}[dtype]
    atol = 1e-4 if dtype == O.F32 else 2e-2
    return atol + ulp * np.abs(ref)


def qref(*args, rounding=O.REF_DECODE, **kw):
    """The oracle's quantized SDPA with the reference's arithmetic (scores
    stored in the query dtype, softmax(precise: false) computed in that
    dtype with its weights stored in it; REF_CHUNK also dequantizes K/V to
    the dtype first) and the per-output rounding bound."""
    return O.quantized_sdpa(*args, rounding=rounding, bound=True, **kw)


def qattn_tol(dtype: int, ref: np.ndarray, wb: np.ndarray) -> np.ndarray:
    """Tolerance against the reference-rounded oracle: attn_tol plus the
    oracle's rounding bound wb, i.e. what the reference's roundings can move
    each output away from the exact softmax of its rounded scores: the
    softmax computed and stored in the dtype (sum_t |w_t - p_t| |v_t|; the
    kernels compute it in fp32 on the rounded scores, since rounding the
    weights as the reference does needs the row's final max and normaliser
    before any P.V, i.e. a second pass over the tokens), and scores within
    fp32 accumulation error of a dtype rounding boundary, which any fp32
    implementation (the reference's included) may round either way."""
    return attn_tol(dtype, ref) + wb


def qref_flip(*args, rounding=O.REF_DECODE, **kw):
    """The oracle's quantized SDPA with the reference's arithmetic and its
    score-boundary term alone: the bound for the reference-softmax path,
    which reproduces the reference's weights from the stored scores, so that
    only a score that an fp32 accumulation rounds to the other side of a
    dtype rounding boundary (either side is as right as the other) moves it."""
    return O.quantized_sdpa(*args, rounding=rounding, flip=True, **kw)


def assert_refclose(got, ref, fb, dtype, ctx=""):
    """Reference-softmax path against the oracle: 2e-2 (1e-4 for f32) + 1 ulp
    + the score-boundary term fb."""
    assert_within(got, ref, attn_tol(dtype, ref) + fb, ctx, fb)


def assert_within(got, ref, tol, ctx="", wb=None):
    """Element-wise |got - ref| <= tol, reporting the worst element (index,
    values, tolerance, the rounding bound there) instead of whole arrays."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    excess = np.abs(got - ref) - np.asarray(tol)
    if not (excess <= 0).all():
        i = np.unravel_index(np.nanargmax(np.where(np.isnan(excess), np.inf, excess)),
                             excess.shape)
        extra = f" bound {np.asarray(wb)[i]:.4g}" if wb is not None else ""
        raise AssertionError(
            f"{ctx}: {(~(excess <= 0)).sum()} of {excess.size} outside tolerance; worst at {i}: "
            f"got {got[i]:.6g} ref {ref[i]:.6g} err {abs(got[i] - ref[i]):.4g} "
            f"tol {np.asarray(tol)[i]:.4g}{extra}; max err {np.nanmax(np.abs(got - ref)):.4g}")


def assert_qclose(got, ref, wb, dtype, ctx=""):
    """assert_within against the reference-rounded oracle (qattn_tol)."""
    assert_within(got, ref, qattn_tol(dtype, ref, wb), ctx, wb)


class _Options:
    """The library's dispatch options as attributes, so that
    monkeypatch.setattr(OPTIONS, "generic_attention", 1) sets one for a
    test and restores it at teardown."""

    def __getattr__(self, name):
        return vkv.get_option(name)

    def __setattr__(self, name, value):
        vkv.set_option(name, value)


OPTIONS = _Options()

