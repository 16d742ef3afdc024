"""Helpers shared by the GPU parity tests: numpy <-> torch-on-HIP moves that
keep bf16/f16 as exact bit patterns, seeded inputs, and tolerances."""
import numpy as np
import torch

import oracle as O

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
