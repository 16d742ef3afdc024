"""Python mirror of the vmlx-swift KV-cache surface over libvkv.so (C ABI).

The engine itself is C++/HIP (``csrc/``); this module is a thin ctypes
binding whose classes keep the reference's names and argument meaning so
that tests read like the reference's own (``KVCacheSimple``,
``RotatingKVCache``, ``QuantizedKVCache``, ``PagedCacheManager``,
``quantized`` / ``dequantized``, ``scaled_dot_product_attention``,
``quantized_scaled_dot_product_attention``).  Device arrays are torch
tensors on the HIP device (torch is the allocator and stream provider only).

The library must be built (``make -C vmlx-swift_amd``); importing this
module without it raises instead of falling back to any CPU path.
"""
from __future__ import annotations

import ctypes as C
import os
import struct
from typing import Optional, Sequence

HERE = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.dirname(HERE)
LIB_PATH = os.path.join(PKG, "libvkv.so")

F32, F16, BF16, U32, I32, U8, BOOL = 0, 1, 2, 3, 4, 5, 6
MASK_NONE, MASK_CAUSAL, MASK_ARRAY = 0, 1, 2
CACHE_SIMPLE, CACHE_ROTATING, CACHE_QUANTIZED = 0, 1, 2
CACHE_COMPILABLE, CACHE_COMPILABLE_ROTATING = 3, 4
CACHE_TURBOQUANT = 5
CACHE_COMPILABLE_TURBOQUANT = 6
VIEW_KEYS_ONLY = 1


class VKVError(RuntimeError):
    pass


class Array(C.Structure):
    _fields_ = [("data", C.c_void_p), ("dtype", C.c_int32), ("ndim", C.c_int32),
                ("shape", C.c_int64 * 4), ("strides", C.c_int64 * 4)]


# the bytes of an Array (data, dtype, ndim, shape[4], strides[4]): one pack
# and one copy build a descriptor about 3x faster than field assignments,
# which dominate a decode step's host time at small shapes
_ARRAY_BYTES = struct.Struct("<qii4q4q")
assert _ARRAY_BYTES.size == C.sizeof(Array)


class PagedView(C.Structure):
    _fields_ = [("base", C.c_void_p), ("dtype", C.c_int32), ("bits", C.c_int32),
                ("group_size", C.c_int32), ("n_kv_heads", C.c_int32), ("head_dim", C.c_int32),
                ("v_head_dim", C.c_int32), ("block_size", C.c_int32), ("flags", C.c_int32),
                ("block_bytes", C.c_int64), ("head_bytes", C.c_int64),
                ("block_table", C.c_void_p), ("table_stride", C.c_int32),
                ("seq_lens", C.c_void_p), ("n_seqs", C.c_int32), ("max_len", C.c_int32)]


class TQEncoded(C.Structure):
    """vkv_tq_encoded: EncodedKeys / EncodedValues as device arrays."""
    _fields_ = [("indices", Array), ("qjl", Array), ("res_norms", Array), ("vec_norms", Array),
                ("sink", Array), ("tail", Array), ("shape", C.c_int32 * 4),
                ("index_bits", C.c_int32), ("seed", C.c_int32)]


class TQInfo(C.Structure):
    _fields_ = [("phase", C.c_int32), ("has_encoded", C.c_int32), ("prefix_tokens", C.c_int64),
                ("window_tokens", C.c_int64), ("key_bits", C.c_int32), ("value_bits", C.c_int32),
                ("sink_tokens", C.c_int32), ("residual_tokens", C.c_int32)]


class CacheParams(C.Structure):
    _fields_ = [("kind", C.c_int32), ("step", C.c_int32), ("max_size", C.c_int32),
                ("keep", C.c_int32), ("group_size", C.c_int32), ("bits", C.c_int32)]


class PoolParams(C.Structure):
    _fields_ = [("num_blocks", C.c_int32), ("block_size", C.c_int32), ("n_layers", C.c_int32),
                ("n_kv_heads", C.c_int32), ("head_dim", C.c_int32), ("v_head_dim", C.c_int32),
                ("dtype", C.c_int32), ("bits", C.c_int32), ("group_size", C.c_int32),
                ("flags", C.c_int32)]


class PrefixStats(C.Structure):
    _fields_ = [("total_blocks", C.c_int64), ("allocated_blocks", C.c_int64),
                ("free_blocks", C.c_int64), ("cache_hits", C.c_int64),
                ("cache_misses", C.c_int64), ("evictions", C.c_int64)]


# Every symbol include/vkv.h declares.
EXPORTS = (
    "vkv_last_error", "vkv_abi_version", "vkv_device_count", "vkv_quantize_affine",
    "vkv_dequantize_affine", "vkv_sdpa", "vkv_quantized_sdpa", "vkv_paged_sdpa",
    "vkv_mla_decode", "vkv_cache_create", "vkv_cache_destroy", "vkv_cache_copy",
    "vkv_cache_update", "vkv_cache_update_quantized", "vkv_cache_offset", "vkv_cache_max_size",
    "vkv_cache_is_trimmable", "vkv_cache_trim", "vkv_cache_capacity", "vkv_cache_state",
    "vkv_cache_set_state", "vkv_cache_meta_state", "vkv_cache_set_meta_state",
    "vkv_cache_make_mask", "vkv_cache_to_quantized", "vkv_cache_to_unquantized",
    "vkv_cache_read_kv", "vkv_pool_create", "vkv_pool_destroy", "vkv_pool_bytes",
    "vkv_pool_view", "vkv_paged_append", "vkv_paged_gather", "vkv_paged_gather_quantized",
    "vkv_pool_copy_blocks", "vkv_prefix_create", "vkv_prefix_destroy", "vkv_prefix_allocate",
    "vkv_prefix_free", "vkv_prefix_release", "vkv_prefix_incref", "vkv_prefix_ref_count", "vkv_prefix_find",
    "vkv_prefix_register", "vkv_prefix_clear", "vkv_prefix_store", "vkv_prefix_fetch",
    "vkv_prefix_stats_get", "vkv_prefix_block_tokens", "vkv_block_hash", "vkv_array_copy",
    "vkv_kernel_timing", "vkv_kernel_timing_read", "vkv_fill_normal",
    "vkv_cache_to_compilable", "vkv_cache_to_compilable_rotating", "vkv_cache_inner_state",
    "vkv_turboquant_to_compilable",
    "vkv_dynamic_slice_update", "vkv_dynamic_slice", "vkv_cache_set_offset",
    "vkv_attention_with_cache_update", "vkv_paged_sdpa_noalloc", "vkv_workspace_release",
    "vkv_quantized_paged_sdpa", "vkv_prefix_writable", "vkv_prompt_cache_save",
    "vkv_prompt_cache_load", "vkv_prompt_cache_save_paged", "vkv_prompt_cache_load_paged",
    "vkv_disk_hash_tokens", "vkv_disk_cache_save", "vkv_disk_cache_load", "vkv_cache_kind",
    "vkv_batch_causal_mask", "vkv_turboquant_create", "vkv_turboquant_from_simple",
    "vkv_turboquant_has_compressible_middle", "vkv_turboquant_info", "vkv_turboquant_encoded",
    "vkv_turboquant_window", "vkv_turboquant_restore_compressed",
    "vkv_turboquant_restore_decoded", "vkv_tq_tables", "vkv_set_option", "vkv_get_option",
    "vkv_turboquant_write_pool", "vkv_cache_update_quantized_tuples",
)
TIME_DECODE, TIME_MLA, TIME_FDECODE, TIME_TQ_ENCODE, TIME_TQ_DECODE, TIME_APPEND = 0, 1, 2, 3, 4, 5

_lib = None


def lib():
    """Load libvkv.so (raises when it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise VKVError(f"{LIB_PATH} is missing: build it with `make -C {PKG}`")
        L = C.CDLL(LIB_PATH)
        L.vkv_last_error.restype = C.c_char_p
        for name in EXPORTS:
            f = getattr(L, name)
            if name != "vkv_last_error":
                f.restype = C.c_int
        _lib = L
    return _lib


def _chk(rc):
    if rc != 0:
        raise VKVError(lib().vkv_last_error().decode())


# ----------------------------------------------------------------- tensors
def _torch():
    import torch

    return torch


_DTYPE_CODES = {}


def _dtype_code(t) -> int:
    if not _DTYPE_CODES:
        torch = _torch()
        _DTYPE_CODES.update({torch.float32: F32, torch.float16: F16, torch.bfloat16: BF16,
                             torch.int32: I32, torch.uint8: U8, torch.bool: BOOL})
    return _DTYPE_CODES[t.dtype]


def arr(t, dtype: Optional[int] = None) -> Array:
    """vkv_array describing a torch tensor (no copy)."""
    nd = t.dim()
    if nd > 4:
        raise ValueError(f"arrays have at most 4 dims, got {nd}")
    pad = (0,) * (4 - nd)
    return Array.from_buffer_copy(_ARRAY_BYTES.pack(
        t.data_ptr() if t.numel() else 0, _dtype_code(t) if dtype is None else dtype, nd,
        *t.shape, *pad, *t.stride(), *pad))


def _torch_dtype(code):
    torch = _torch()
    return {F32: torch.float32, F16: torch.float16, BF16: torch.bfloat16, U32: torch.int32,
            I32: torch.int32, U8: torch.uint8, BOOL: torch.bool}[code]


def stream_ptr(stream=None):
    """The HIP stream handle of `stream`, or of the current stream: through
    torch's raw accessor where it has one (a Stream object costs ~3 us to
    build, most of a small decode call's host time)."""
    torch = _torch()
    if stream is None:
        raw = getattr(torch._C, "_cuda_getCurrentRawStream", None)
        if raw is not None:
            return C.c_void_p(raw(torch._C._cuda_getDevice()))
        stream = torch.cuda.current_stream()
    return C.c_void_p(stream.cuda_stream)


def to_torch(a: Array, stream=None):
    """Materialize a library-owned array into a fresh contiguous tensor.
    u32 arrays come back as int32 tensors with the same bits."""
    torch = _torch()
    shape = tuple(a.shape[i] for i in range(a.ndim))
    out = torch.empty(shape, dtype=_torch_dtype(a.dtype), device="cuda")
    if out.numel():
        dst = arr(out, a.dtype)
        _chk(lib().vkv_array_copy(C.byref(a), C.byref(dst), stream_ptr(stream)))
    return out


# ------------------------------------------------------------------- ops
OPTIONS = {"generic_attention": 0, "decode_waves": 1, "mla_splits": 2, "fdecode_waves": 3,
           "gather_tokens": 4, "reference_softmax": 5, "separate_token_write": 6}


def set_option(name: str, value: int):
    """vkv_set_option: process-wide dispatch options (generic_attention,
    decode_waves, mla_splits)."""
    _chk(lib().vkv_set_option(OPTIONS[name], C.c_int64(int(value))))


def get_option(name: str) -> int:
    v = C.c_int64()
    _chk(lib().vkv_get_option(OPTIONS[name], C.byref(v)))
    return v.value


def batch_causal_mask(n: int, offsets, effective_key_lens=None, window_size=None, stream=None):
    """createBatchCausalMask(queryLen:offsets:effectiveKeyLens:windowSize:)
    (BatchEngine/BatchMask.swift:44-115): a bool tensor [B, 1, n, maxTotal]."""
    torch = _torch()
    B = len(offsets)
    offs = (C.c_int32 * max(1, B))(*offsets)
    kls = None
    if effective_key_lens is not None:
        if len(effective_key_lens) != B:
            raise VKVError(f"effectiveKeyLens.count {len(effective_key_lens)} must equal "
                           f"offsets.count {B}")
        kls = (C.c_int32 * max(1, B))(*effective_key_lens)
    win = -1 if window_size is None else int(window_size)
    mt = C.c_int32()
    _chk(lib().vkv_batch_causal_mask(n, offs, kls, B, win, None, C.c_int64(0), None, C.byref(mt)))
    out = torch.empty((B, 1, n, mt.value), dtype=torch.bool, device="cuda")
    if out.numel():
        _chk(lib().vkv_batch_causal_mask(n, offs, kls, B, win, C.c_void_p(out.data_ptr()),
                                         C.c_int64(out.numel()), stream_ptr(stream),
                                         C.byref(mt)))
    return out


def quantized(w, group_size: int = 64, bits: int = 4, stream=None):
    """mlx `quantized(_:groupSize:bits:)` (Source/MLX/Ops.swift:2368-2391),
    affine mode: returns (wq int32-as-u32, scales, biases)."""
    torch = _torch()
    D = w.shape[-1]
    wq = torch.empty(w.shape[:-1] + (D * bits // 32,), dtype=torch.int32, device=w.device)
    sc = torch.empty(w.shape[:-1] + (D // group_size,), dtype=w.dtype, device=w.device)
    bi = torch.empty_like(sc)
    a_wq, a_sc, a_bi = arr(wq, U32), arr(sc), arr(bi)
    _chk(lib().vkv_quantize_affine(C.byref(arr(w)), group_size, bits, C.byref(a_wq),
                                   C.byref(a_sc), C.byref(a_bi), stream_ptr(stream)))
    return wq, sc, bi


def dequantized(wq, scales, biases, group_size: int = 64, bits: int = 4, stream=None):
    """mlx `dequantized(...)` (Source/MLX/Ops.swift:1146-1163), affine mode."""
    torch = _torch()
    D = wq.shape[-1] * 32 // bits
    out = torch.empty(wq.shape[:-1] + (D,), dtype=scales.dtype, device=wq.device)
    a_out = arr(out)
    _chk(lib().vkv_dequantize_affine(C.byref(arr(wq, U32)), C.byref(arr(scales)),
                                     C.byref(arr(biases)), group_size, bits, C.byref(a_out),
                                     stream_ptr(stream)))
    return out


def _as_array(x):
    """A library-owned Array passes through; a tensor is described."""
    return x if isinstance(x, Array) else arr(x)


def _sinks_arg(sinks):
    return None if sinks is None else C.byref(arr(sinks))


def _mask_args(mask):
    if mask is None:
        return MASK_NONE, None
    if isinstance(mask, str):
        assert mask == "causal"
        return MASK_CAUSAL, None
    return MASK_ARRAY, C.byref(_as_array(mask))


def scaled_dot_product_attention(queries, keys, values, scale: float, mask=None, stream=None,
                                 out=None, sinks=None):
    """MLXFast.scaledDotProductAttention (Source/MLX/MLXFast.swift:203-218).
    keys, values and an array mask may be tensors or library-owned Arrays
    (the views a cache returns); `out` may be given (nothing is allocated
    then, as a captured HIP graph needs); `sinks` is an optional [Hq]
    tensor of attention-sink logits."""
    torch = _torch()
    B, Hq, L, _ = queries.shape
    a_k, a_v = _as_array(keys), _as_array(values)
    if out is None:
        out = torch.empty((B, Hq, L, a_v.shape[3]), dtype=queries.dtype, device=queries.device)
    mode, m = _mask_args(mask)
    a_out = arr(out)
    _chk(lib().vkv_sdpa(C.byref(arr(queries)), C.byref(a_k), C.byref(a_v),
                        C.c_float(scale), mode, m, _sinks_arg(sinks), C.byref(a_out),
                        stream_ptr(stream)))
    return out


def attention_with_cache_update(queries, keys, values, cache, scale: float, mask=None,
                                stream=None, out=None, sinks=None):
    """attentionWithCacheUpdate (MLXLMCommon/AttentionUtils.swift:77-143):
    updates `cache` (None: no cache) with the new keys/values and attends the
    queries [B, Hq, L, D] over the cached K/V; see
    vkv_attention_with_cache_update for the routing."""
    torch = _torch()
    B, Hq, L, _ = queries.shape
    if out is None:
        dv = values.shape[3]
        out = torch.empty((B, Hq, L, dv), dtype=queries.dtype, device=queries.device)
    mode, m = _mask_args(mask)
    a_out = arr(out)
    _chk(lib().vkv_attention_with_cache_update(
        C.byref(arr(queries)), C.byref(arr(keys)), C.byref(arr(values)),
        cache._h if cache is not None else None, C.c_float(scale), mode, m, _sinks_arg(sinks),
        C.byref(a_out), stream_ptr(stream)))
    return out


def quantized_scaled_dot_product_attention(queries, quantized_keys, quantized_values,
                                           scale: float, mask=None, group_size: int = 64,
                                           bits: int = 8, stream=None):
    """quantizedScaledDotProductAttention (MLXLMCommon/KVCache.swift:1909-1997)
    over reference-layout tuples (wq, scales, biases)."""
    torch = _torch()
    out = torch.empty_like(queries)
    (kw, ks, kb), (vw, vs, vb) = quantized_keys, quantized_values
    mode, m = _mask_args(mask)
    a_out = arr(out)
    _chk(lib().vkv_quantized_sdpa(
        C.byref(arr(queries)), C.byref(arr(kw, U32)), C.byref(arr(ks)), C.byref(arr(kb)),
        C.byref(arr(vw, U32)), C.byref(arr(vs)), C.byref(arr(vb)), group_size, bits,
        C.c_float(scale), mode, m, C.byref(a_out), stream_ptr(stream)))
    return out


def paged_attention(queries, view: PagedView, scale: float, stream=None, out=None,
                    noalloc: bool = False):
    """Decode attention over paged KV: queries [n_seqs, Hq, D].  With
    noalloc=True the call goes to vkv_paged_sdpa_noalloc (split-K partials in
    the library's fixed device scratch; pass `out` to allocate nothing on
    this side either)."""
    torch = _torch()
    if out is None:
        out = torch.empty((queries.shape[0], queries.shape[1], view.v_head_dim),
                          dtype=queries.dtype, device=queries.device)
    a_out = arr(out)
    fn = lib().vkv_paged_sdpa_noalloc if noalloc else lib().vkv_paged_sdpa
    _chk(fn(C.byref(arr(queries)), C.byref(view), C.c_float(scale), C.byref(a_out),
            stream_ptr(stream)))
    return out


def quantized_paged_attention(queries, view: PagedView, scale: float, mask=None, stream=None,
                              out=None):
    """quantizedScaledDotProductAttention (KVCache.swift:1909-1997) over the
    paged view updateQuantized returned: queries [n_seqs, Hq, L, D], any L."""
    torch = _torch()
    if out is None:
        out = torch.empty(tuple(queries.shape[:3]) + (view.v_head_dim,), dtype=queries.dtype,
                          device=queries.device)
    mode, m = _mask_args(mask)
    a_out = arr(out)
    _chk(lib().vkv_quantized_paged_sdpa(C.byref(arr(queries)), C.byref(view), C.c_float(scale),
                                        mode, m, C.byref(a_out), stream_ptr(stream)))
    return out


def workspace_release(stream=None) -> int:
    """Free the attention workspace of a stream, outgrown buffers included
    (only once no captured graph that used the stream is replayed again);
    returns the bytes released."""
    n = C.c_int64()
    _chk(lib().vkv_workspace_release(stream_ptr(stream), C.byref(n)))
    return n.value


def mla_decode(queries, view: PagedView, scale: float, stream=None):
    torch = _torch()
    out = torch.empty((queries.shape[0], queries.shape[1], view.v_head_dim), dtype=queries.dtype,
                      device=queries.device)
    a_out = arr(out)
    _chk(lib().vkv_mla_decode(C.byref(arr(queries)), C.byref(view), C.c_float(scale),
                              C.byref(a_out), stream_ptr(stream)))
    return out


def kernel_timing(enable: bool):
    """Start (True) or stop recording event pairs around the decode, MLA,
    TurboQuant and pool-append kernels (a measurement aid; see
    vkv_kernel_timing)."""
    _chk(lib().vkv_kernel_timing(C.c_int32(1 if enable else 0)))


def kernel_timing_read(kind: int):
    """(total milliseconds, launches) recorded for a kind (TIME_DECODE,
    TIME_MLA, ...) since the last read; waits for those launches."""
    ms = C.c_double()
    n = C.c_int32()
    _chk(lib().vkv_kernel_timing_read(C.c_int32(kind), C.byref(ms), C.byref(n)))
    return ms.value, n.value


def fill_normal(t, seed: int, std: float = 1.0, stream=None):
    _chk(lib().vkv_fill_normal(C.c_void_p(t.data_ptr()), _dtype_code(t), t.numel(),
                               C.c_uint64(seed), C.c_float(std), stream_ptr(stream)))
    return t


def block_hash(parent_hash: Optional[str], tokens: Sequence[int], model_key: Optional[str] = None,
               media_salt: Optional[str] = None) -> str:
    """CacheBlock.computeBlockHash (Cache/CacheBlock.swift:110-146)."""
    toks = (C.c_int64 * max(1, len(tokens)))(*tokens)
    out = C.create_string_buffer(65)
    _chk(lib().vkv_block_hash(
        parent_hash.encode() if parent_hash is not None else None, toks, len(tokens),
        model_key.encode() if model_key is not None else None,
        media_salt.encode() if media_salt is not None else None, out))
    return out.value.decode()


# ------------------------------------------------------------------ caches
class _Cache:
    def __init__(self, params: CacheParams, handle=None):
        self._h = C.c_void_p()
        if handle is not None:
            self._h = handle
        else:
            _chk(lib().vkv_cache_create(C.byref(params), C.byref(self._h)))

    def __del__(self):
        if getattr(self, "_h", None) and _lib is not None:
            _lib.vkv_cache_destroy(self._h)
            self._h = None

    @property
    def kind(self) -> int:
        """The cache's class (CACHE_*), vkv_cache_kind."""
        v = C.c_int32()
        _chk(lib().vkv_cache_kind(self._h, C.byref(v)))
        return v.value

    @property
    def offset(self) -> int:
        v = C.c_int64()
        _chk(lib().vkv_cache_offset(self._h, C.byref(v)))
        return v.value

    @offset.setter
    def offset(self, value: int):
        _chk(lib().vkv_cache_set_offset(self._h, C.c_int64(value)))

    @property
    def max_size(self) -> Optional[int]:
        v = C.c_int64()
        _chk(lib().vkv_cache_max_size(self._h, C.byref(v)))
        return None if v.value < 0 else v.value

    @property
    def capacity(self) -> int:
        v = C.c_int64()
        _chk(lib().vkv_cache_capacity(self._h, C.byref(v)))
        return v.value

    @property
    def is_trimmable(self) -> bool:
        v = C.c_int32()
        _chk(lib().vkv_cache_is_trimmable(self._h, C.byref(v)))
        return bool(v.value)

    def trim(self, n: int) -> int:
        v = C.c_int64()
        _chk(lib().vkv_cache_trim(self._h, n, C.byref(v)))
        return v.value

    def update(self, keys, values, stream=None):
        """update(keys:values:) -> (keys, values) as library-owned views."""
        ok, ov = Array(), Array()
        _chk(lib().vkv_cache_update(self._h, C.byref(arr(keys)), C.byref(arr(values)),
                                    stream_ptr(stream), C.byref(ok), C.byref(ov)))
        return ok, ov

    def state_views(self, stream=None):
        arrs = (Array * 6)()
        n = C.c_int32()
        _chk(lib().vkv_cache_state(self._h, stream_ptr(stream), arrs, C.byref(n)))
        return [arrs[i] for i in range(n.value)]

    @property
    def state(self):
        """state getter, materialized as torch tensors."""
        return [to_torch(a) for a in self.state_views()]

    @state.setter
    def state(self, tensors):
        kinds = [U32 if (t.dtype == _torch().int32) else None for t in tensors]
        arrs = (Array * max(1, len(tensors)))(*[arr(t, k) for t, k in zip(tensors, kinds)])
        _chk(lib().vkv_cache_set_state(self._h, arrs, len(tensors), stream_ptr()))

    @property
    def meta_state(self):
        buf = C.create_string_buffer(4096)
        n = C.c_int32()
        _chk(lib().vkv_cache_meta_state(self._h, buf, 4096, C.byref(n)))
        parts = buf.raw.split(b"\0")
        return [p.decode() for p in parts[: n.value]]

    @meta_state.setter
    def meta_state(self, strings):
        arrs = (C.c_char_p * max(1, len(strings)))(*[s.encode() for s in strings])
        _chk(lib().vkv_cache_set_meta_state(self._h, arrs, len(strings)))

    def make_mask(self, n: int, window_size: Optional[int] = None, return_array: bool = False):
        """makeMask(n:windowSize:returnArray:) -> ('none'|'causal'|tensor)."""
        mode = C.c_int32()
        m = Array()
        _chk(lib().vkv_cache_make_mask(self._h, n, window_size or 0, int(return_array),
                                       stream_ptr(), C.byref(mode), C.byref(m)))
        if mode.value == MASK_NONE:
            return "none"
        if mode.value == MASK_CAUSAL:
            return "causal"
        return to_torch(m)

    def read_kv(self):
        k, v = Array(), Array()
        _chk(lib().vkv_cache_read_kv(self._h, stream_ptr(), C.byref(k), C.byref(v)))
        return to_torch(k), to_torch(v)

    def copy(self):
        h = C.c_void_p()
        _chk(lib().vkv_cache_copy(self._h, stream_ptr(), C.byref(h)))
        new = object.__new__(type(self))
        _Cache.__init__(new, None, handle=h)
        return new


class KVCacheSimple(_Cache):
    """KVCacheSimple (MLXLMCommon/KVCache.swift:452-596)."""

    def __init__(self, step: int = 256):
        super().__init__(CacheParams(CACHE_SIMPLE, step, 0, 0, 0, 0))

    def to_quantized(self, group_size: int = 64, bits: int = 4):
        h = C.c_void_p()
        _chk(lib().vkv_cache_to_quantized(self._h, group_size, bits, stream_ptr(), C.byref(h)))
        q = object.__new__(QuantizedKVCache)
        _Cache.__init__(q, None, handle=h)
        q.group_size, q.bits = group_size, bits
        return q


class RotatingKVCache(_Cache):
    """RotatingKVCache (MLXLMCommon/KVCache.swift:605-958)."""

    def __init__(self, max_size: int, keep: int = 0, step: int = 256):
        super().__init__(CacheParams(CACHE_ROTATING, step, max_size, keep, 0, 0))


class _FixedBuffer(_Cache):
    def inner_state(self):
        """innerState: the fixed buffers and the int32 [1] device counters,
        as library-owned arrays (write them in place only)."""
        arrs = (Array * 4)()
        n = C.c_int32()
        _chk(lib().vkv_cache_inner_state(self._h, arrs, C.byref(n)))
        return [arrs[i] for i in range(n.value)]


def _wrap(cls, h):
    new = object.__new__(cls)
    _Cache.__init__(new, None, handle=h)
    return new


class CompilableKVCache(_FixedBuffer):
    """CompilableKVCache (MLXLMCommon/CompilableKVCache.swift:40-262): fixed
    [B, H, max_length, D] buffers, write offset in device memory; update
    returns the whole buffers and make_mask an array mask built on the
    device, so a decode step can be captured in a HIP graph."""

    def __init__(self, max_length: int = 4096, step: int = 256):
        super().__init__(CacheParams(CACHE_COMPILABLE, step, max_length, 0, 0, 0))

    @classmethod
    def from_cache(cls, cache, max_length: int = 4096):
        """CompilableKVCache(from:maxLength:) (CompilableKVCache.swift:62-86)."""
        h = C.c_void_p()
        _chk(lib().vkv_cache_to_compilable(cache._h, C.c_int64(max_length), stream_ptr(),
                                           C.byref(h)))
        return _wrap(cls, h)


class CompilableRotatingKVCache(_FixedBuffer):
    """CompilableRotatingKVCache (BatchEngine/CompilableRotatingKVCache.swift:
    1-265): a RotatingKVCache with maxSize buffers allocated once and its ring
    index and offset in device memory."""

    def __init__(self, max_size: int, keep: int = 0, step: int = 256):
        super().__init__(CacheParams(CACHE_COMPILABLE_ROTATING, step, max_size, keep, 0, 0))

    @classmethod
    def from_rotating(cls, rotating):
        """CompilableRotatingKVCache(from:) (CompilableRotatingKVCache.swift:91-150)."""
        h = C.c_void_p()
        _chk(lib().vkv_cache_to_compilable_rotating(rotating._h, stream_ptr(), C.byref(h)))
        return _wrap(cls, h)


def dynamic_slice_update(dst, update, start, axis: int, stream=None):
    """dynamicSliceUpdate (MLXLMCommon/DynamicSlice.swift:50-71), in place:
    dst[..., s + i, ...] = update[..., i, ...] along axis, with s the int32
    in the device tensor `start` (clamped so the update fits)."""
    a_d, a_u = arr(dst), arr(update)
    _chk(lib().vkv_dynamic_slice_update(C.byref(a_d), C.byref(a_u), C.c_void_p(start.data_ptr()),
                                        axis, stream_ptr(stream)))
    return dst


def dynamic_slice(src, start, axis: int, size: int, stream=None):
    """dynamicSlice (MLXLMCommon/DynamicSlice.swift:21-48): src[..., s : s + size, ...]
    along axis with s read from the device tensor `start`."""
    torch = _torch()
    ax = axis % src.dim()
    shape = list(src.shape)
    shape[ax] = size
    out = torch.empty(shape, dtype=src.dtype, device=src.device)
    a_s, a_o = arr(src), arr(out)
    _chk(lib().vkv_dynamic_slice(C.byref(a_s), C.c_void_p(start.data_ptr()), axis, C.byref(a_o),
                                 stream_ptr(stream)))
    return out


class QuantizedKVCache(_Cache):
    """QuantizedKVCache (MLXLMCommon/KVCache.swift:961-1221)."""

    def __init__(self, group_size: int = 64, bits: int = 8):
        super().__init__(CacheParams(CACHE_QUANTIZED, 256, 0, 0, group_size, bits))
        self.group_size, self.bits = group_size, bits

    def update_quantized(self, keys, values, stream=None) -> PagedView:
        v = PagedView()
        _chk(lib().vkv_cache_update_quantized(self._h, C.byref(arr(keys)), C.byref(arr(values)),
                                              stream_ptr(stream), C.byref(v)))
        return v

    def update_quantized_tuples(self, keys, values, stream=None):
        """updateQuantized(keys:values:) -> ((wq, scales, biases), (wq,
        scales, biases)) as library-owned [B, H, offset, *] views
        (vkv_cache_update_quantized_tuples; to_torch materializes one)."""
        out = (Array * 6)()
        _chk(lib().vkv_cache_update_quantized_tuples(self._h, C.byref(arr(keys)),
                                                     C.byref(arr(values)), stream_ptr(stream),
                                                     out))
        return (out[0], out[1], out[2]), (out[3], out[4], out[5])

    def to_unquantized(self):
        h = C.c_void_p()
        _chk(lib().vkv_cache_to_unquantized(self._h, stream_ptr(), C.byref(h)))
        s = object.__new__(KVCacheSimple)
        _Cache.__init__(s, None, handle=h)
        return s


class TurboQuantKVCache(_Cache):
    """TurboQuantKVCache (TurboQuant/TurboQuantKVCache.swift:70-671)."""
    DEFAULT_RESIDUAL_TOKENS = 64
    MINIMUM_COMPRESSED_TOKENS = 8

    def __init__(self, key_bits: int = 3, value_bits: int = 3, sink_tokens: int = 4,
                 residual_tokens: int = 64, handle=None):
        self._h = C.c_void_p()
        if handle is not None:
            self._h = handle
        else:
            _chk(lib().vkv_turboquant_create(key_bits, value_bits, sink_tokens, residual_tokens,
                                             C.byref(self._h)))

    @staticmethod
    def from_simple_cache(source: "KVCacheSimple", key_bits: int, value_bits: int,
                          sink_tokens: int = 4, residual_tokens: int = 64, stream=None):
        h = C.c_void_p()
        _chk(lib().vkv_turboquant_from_simple(source._h, key_bits, value_bits, sink_tokens,
                                              residual_tokens, stream_ptr(stream), C.byref(h)))
        return TurboQuantKVCache(handle=h)

    @staticmethod
    def has_compressible_middle(token_count: int, sink_tokens: int = 4,
                                residual_tokens: int = 64, minimum: int = 8) -> bool:
        out = C.c_int32()
        _chk(lib().vkv_turboquant_has_compressible_middle(C.c_int64(token_count), sink_tokens,
                                                          residual_tokens, minimum, C.byref(out)))
        return bool(out.value)

    @property
    def info(self) -> dict:
        i = TQInfo()
        _chk(lib().vkv_turboquant_info(self._h, C.byref(i)))
        return {f: getattr(i, f) for f, _ in TQInfo._fields_}

    @property
    def phase(self) -> str:
        return "compressed" if self.info["phase"] else "fill"

    def encoded_views(self):
        k, v = TQEncoded(), TQEncoded()
        _chk(lib().vkv_turboquant_encoded(self._h, C.byref(k), C.byref(v)))
        return k, v

    def encoded(self):
        """(compressedKeys, compressedValues) as dicts of fresh tensors."""
        def rec(e):
            get = lambda a: to_torch(a) if a.ndim else None
            return {"indices": get(e.indices), "qjl": get(e.qjl), "res_norms": get(e.res_norms),
                    "vec_norms": get(e.vec_norms), "sink": get(e.sink), "tail": get(e.tail),
                    "shape": list(e.shape), "index_bits": e.index_bits, "seed": e.seed}
        k, v = self.encoded_views()
        return rec(k), rec(v)

    def write_pool(self, pool: "PagedPool", layer: int, slots, first: int = 0, n=None,
                   stream=None):
        """Write tokens [first, first + n) of the K/V update() returns (all of
        them by default) into pool slots (device int32 [B * n]): the cache
        as pool pages (vkv_turboquant_write_pool)."""
        if n is None:
            n = self.offset - first
        if slots.dtype != _torch().int32 or not slots.is_contiguous() or slots.numel() < n:
            raise VKVError("slots must be a contiguous int32 device tensor of B * n entries")
        _chk(lib().vkv_turboquant_write_pool(self._h, pool._h, layer,
                                             C.c_void_p(slots.data_ptr()), C.c_int64(first),
                                             C.c_int64(n), stream_ptr(stream)))

    def window_state(self):
        k, v, p = Array(), Array(), C.c_int32()
        _chk(lib().vkv_turboquant_window(self._h, C.byref(k), C.byref(v), C.byref(p)))
        return (to_torch(k), to_torch(v)) if p.value else None

    @staticmethod
    def _record(r: dict) -> TQEncoded:
        e = TQEncoded()
        e.indices = arr(r["indices"], U32)
        if r.get("qjl") is not None:
            e.qjl = arr(r["qjl"], U32)
        if r.get("res_norms") is not None:
            e.res_norms = arr(r["res_norms"])
        e.vec_norms = arr(r["vec_norms"])
        if r.get("sink") is not None:
            e.sink = arr(r["sink"])
        if r.get("tail") is not None:
            e.tail = arr(r["tail"])
        for i in range(4):
            e.shape[i] = r["shape"][i]
        e.index_bits = r["index_bits"]
        e.seed = r.get("seed", 42)
        return e

    def restore_compressed(self, keys: dict, values: dict, source_offset: int,
                           window_keys=None, window_values=None, stream=None):
        """restoreCompressed(encodedKeys:encodedValues:sourceOffset:windowKeys:
        windowValues:); records as returned by encoded()."""
        ek, ev = self._record(keys), self._record(values)
        wk = C.byref(arr(window_keys)) if window_keys is not None else None
        wv = C.byref(arr(window_values)) if window_values is not None else None
        _chk(lib().vkv_turboquant_restore_compressed(self._h, C.byref(ek), C.byref(ev),
                                                     C.c_int64(source_offset), wk, wv,
                                                     stream_ptr(stream)))

    def restore_from_decoded(self, keys, values, source_offset: int, stream=None):
        _chk(lib().vkv_turboquant_restore_decoded(self._h, C.byref(arr(keys)),
                                                  C.byref(arr(values)), C.c_int64(source_offset),
                                                  stream_ptr(stream)))


class CompilableTurboQuantKVCache(TurboQuantKVCache):
    """CompilableTurboQuantKVCache (BatchEngine/CompilableTurboQuantKVCache.
    swift:57-294): a compressed TurboQuantKVCache whose window writes go to
    the offset in device memory; update returns the whole unified buffers and
    make_mask an array mask over them, so a decode step can be captured in a
    HIP graph."""

    @classmethod
    def from_turboquant(cls, tq: TurboQuantKVCache, stream=None):
        """CompilableTurboQuantKVCache(from:) (:110-160); tq must be compressed."""
        h = C.c_void_p()
        _chk(lib().vkv_turboquant_to_compilable(tq._h, stream_ptr(stream), C.byref(h)))
        return cls(handle=h)

    def inner_state(self):
        """innerState (:286-293): the unified keys and values, then the int32
        [1] device counters (window write position, offset)."""
        arrs = (Array * 4)()
        n = C.c_int32()
        _chk(lib().vkv_cache_inner_state(self._h, arrs, C.byref(n)))
        return [arrs[i] for i in range(n.value)]


def tq_tables(dim: int, bits: int, seed: int = 42):
    """(rotation signs, Lloyd-Max codebook, QJL matrix) of the codec's
    EncoderState, from the library's host code (no device needed)."""
    import numpy as np
    signs = np.empty(dim, np.float32)
    cb = np.empty(1 << bits, np.float32)
    S = np.empty((dim, dim), np.float32)
    f = lambda a: a.ctypes.data_as(C.c_void_p)
    _chk(lib().vkv_tq_tables(dim, bits, seed, f(signs), f(cb), f(S)))
    return signs, cb, S


# -------------------------------------------------------------------- pool
class PagedPool:
    """Device block pool: [layer][block][kv head] chunks."""

    def __init__(self, num_blocks, block_size, n_layers, n_kv_heads, head_dim, dtype=BF16,
                 bits=0, group_size=64, v_head_dim=0, flags=0):
        self.params = PoolParams(num_blocks, block_size, n_layers, n_kv_heads, head_dim,
                                 v_head_dim, dtype, bits, group_size, flags)
        self._h = C.c_void_p()
        _chk(lib().vkv_pool_create(C.byref(self.params), C.byref(self._h)))

    def __del__(self):
        if getattr(self, "_h", None) and _lib is not None:
            _lib.vkv_pool_destroy(self._h)
            self._h = None

    @property
    def nbytes(self) -> int:
        v = C.c_int64()
        _chk(lib().vkv_pool_bytes(self._h, C.byref(v)))
        return v.value

    def view(self, layer, block_table, seq_lens, max_len) -> PagedView:
        v = PagedView()
        _chk(lib().vkv_pool_view(self._h, layer, C.c_void_p(block_table.data_ptr()),
                                 block_table.stride(0),
                                 C.c_void_p(seq_lens.data_ptr()) if seq_lens is not None else None,
                                 block_table.shape[0], max_len, C.byref(v)))
        v._keep = (block_table, seq_lens)
        return v

    def append(self, layer, keys, values, slot_mapping, stream=None):
        _chk(lib().vkv_paged_append(self._h, layer, C.byref(arr(keys)),
                                    C.byref(arr(values)) if values is not None else None,
                                    C.c_void_p(slot_mapping.data_ptr()), keys.shape[0],
                                    stream_ptr(stream)))

    def copy_blocks(self, src, dst, stream=None):
        n = len(src)
        a = (C.c_int32 * max(1, n))(*src)
        b = (C.c_int32 * max(1, n))(*dst)
        _chk(lib().vkv_pool_copy_blocks(self._h, a, b, n, stream_ptr(stream)))


def paged_gather(view: PagedView, stream=None):
    """Dequant-on-read gather -> (keys, values) [n, Hkv, max_len, D]."""
    torch = _torch()
    dt = _torch_dtype(view.dtype)
    k = torch.zeros((view.n_seqs, view.n_kv_heads, view.max_len, view.head_dim), dtype=dt,
                    device="cuda")
    keys_only = bool(view.flags & VIEW_KEYS_ONLY)
    v = None if keys_only else torch.zeros(
        (view.n_seqs, view.n_kv_heads, view.max_len, view.v_head_dim), dtype=dt, device="cuda")
    ak = arr(k)
    av = arr(v) if v is not None else None
    _chk(lib().vkv_paged_gather(C.byref(view), C.byref(ak), C.byref(av) if av is not None else None,
                                stream_ptr(stream)))
    return k, v


def paged_gather_quantized(view: PagedView, stream=None):
    """Raw affine codes in the reference layout: ((wq, s, b), (wq, s, b))."""
    torch = _torch()
    dt = _torch_dtype(view.dtype)
    n, H, T, D = view.n_seqs, view.n_kv_heads, view.max_len, view.head_dim
    W, G = D * view.bits // 32, D // view.group_size
    outs = []
    for _ in range(2):
        outs += [torch.zeros((n, H, T, W), dtype=torch.int32, device="cuda"),
                 torch.zeros((n, H, T, G), dtype=dt, device="cuda"),
                 torch.zeros((n, H, T, G), dtype=dt, device="cuda")]
    arrs = (Array * 6)(*[arr(t, U32 if i % 3 == 0 else None) for i, t in enumerate(outs)])
    _chk(lib().vkv_paged_gather_quantized(C.byref(view), arrs, stream_ptr(stream)))
    return tuple(outs[:3]), tuple(outs[3:])


# ------------------------------------------------------------ prefix cache
class PagedCacheManager:
    """PagedCacheManager (MLXLMCommon/Cache/PagedCacheManager.swift)."""

    def __init__(self, block_size: int = 64, max_blocks: int = 1000,
                 model_key: Optional[str] = None, pool: Optional[PagedPool] = None):
        self.block_size, self.max_blocks = block_size, max_blocks
        self._pool = pool
        self._h = C.c_void_p()
        _chk(lib().vkv_prefix_create(block_size, max_blocks,
                                     model_key.encode() if model_key is not None else None,
                                     pool._h if pool is not None else None, C.byref(self._h)))

    def __del__(self):
        if getattr(self, "_h", None) and _lib is not None:
            _lib.vkv_prefix_destroy(self._h)
            self._h = None

    def allocate_block(self) -> Optional[int]:
        b = C.c_int32()
        _chk(lib().vkv_prefix_allocate(self._h, C.byref(b)))
        return None if b.value < 0 else b.value

    def free_block(self, block: int):
        _chk(lib().vkv_prefix_free(self._h, block))

    def release(self, blocks: Sequence[int]):
        """CacheCoordinator.release(blocks:): leaves first."""
        a = (C.c_int32 * max(1, len(blocks)))(*blocks)
        _chk(lib().vkv_prefix_release(self._h, a, len(blocks)))

    def incref(self, block: int):
        _chk(lib().vkv_prefix_incref(self._h, block))

    def ref_count(self, block: int) -> int:
        v = C.c_int32()
        _chk(lib().vkv_prefix_ref_count(self._h, block, C.byref(v)))
        return v.value

    def token_count(self, block: int) -> int:
        v = C.c_int32()
        _chk(lib().vkv_prefix_block_tokens(self._h, block, C.byref(v)))
        return v.value

    def find_cached_block(self, hash_: str) -> Optional[int]:
        b = C.c_int32()
        _chk(lib().vkv_prefix_find(self._h, hash_.encode(), C.byref(b)))
        return None if b.value < 0 else b.value

    def register_block(self, block: int, hash_: str):
        _chk(lib().vkv_prefix_register(self._h, block, hash_.encode()))

    def clear(self):
        _chk(lib().vkv_prefix_clear(self._h))

    def store_token_sequence(self, tokens: Sequence[int], n_data_chunks: int,
                             src_blocks: Optional[Sequence[int]] = None,
                             media_salt: Optional[str] = None, stream=None):
        toks = (C.c_int64 * max(1, len(tokens)))(*tokens)
        src = (C.c_int32 * max(1, len(src_blocks)))(*src_blocks) if src_blocks else None
        _chk(lib().vkv_prefix_store(self._h, toks, len(tokens),
                                    media_salt.encode() if media_salt is not None else None,
                                    n_data_chunks, src,
                                    stream_ptr(stream) if self._pool is not None else None))

    def fetch_prefix(self, tokens: Sequence[int], media_salt: Optional[str] = None):
        """-> None or (matched_tokens, remaining_tokens, blocks)."""
        toks = (C.c_int64 * max(1, len(tokens)))(*tokens)
        cap = len(tokens) + 1
        blocks = (C.c_int32 * cap)()
        nb, matched = C.c_int32(), C.c_int64()
        _chk(lib().vkv_prefix_fetch(self._h, toks, len(tokens),
                                    media_salt.encode() if media_salt is not None else None,
                                    blocks, cap, C.byref(nb), C.byref(matched)))
        if nb.value == 0:
            return None
        return matched.value, list(tokens[matched.value:]), [blocks[i] for i in range(nb.value)]

    def writable(self, block: int, stream=None) -> Optional[int]:
        """Copy-on-write before writing into `block` (vkv_prefix_writable):
        the block to write into, or None when the pool has no free block."""
        b = C.c_int32()
        _chk(lib().vkv_prefix_writable(self._h, block,
                                       stream_ptr(stream) if self._pool is not None else None,
                                       C.byref(b)))
        return None if b.value < 0 else b.value

    @property
    def stats(self) -> dict:
        s = PrefixStats()
        _chk(lib().vkv_prefix_stats_get(self._h, C.byref(s)))
        return {f: getattr(s, f) for f, _ in PrefixStats._fields_}


# ----------------------------------------------------------- on-disk formats
def _wrap_handle(h):
    """A library cache handle as the Python class of its kind."""
    k = C.c_int32()
    _chk(lib().vkv_cache_kind(h, C.byref(k)))
    cls = {CACHE_SIMPLE: KVCacheSimple, CACHE_ROTATING: RotatingKVCache,
           CACHE_QUANTIZED: QuantizedKVCache, CACHE_TURBOQUANT: TurboQuantKVCache,
           CACHE_COMPILABLE_TURBOQUANT: CompilableTurboQuantKVCache}.get(k.value,
                                                                                     _Cache)
    obj = object.__new__(cls)
    _Cache.__init__(obj, None, handle=h)
    return obj


def _meta_args(metadata):
    items = list((metadata or {}).items())
    keys = (C.c_char_p * max(1, len(items)))(*[k.encode() for k, _ in items])
    vals = (C.c_char_p * max(1, len(items)))(*[v.encode() for _, v in items])
    return keys, vals, len(items)


def _meta_out(call):
    """Runs call(buf, len, n_ptr) twice (count, then fill) -> dict."""
    n = C.c_int32()
    call(None, C.c_int64(0), C.byref(n))
    buf = C.create_string_buffer(1 << 16)
    while True:
        try:
            call(buf, C.c_int64(len(buf)), C.byref(n))
            break
        except VKVError as e:
            if "too small" not in str(e):
                raise
            buf = C.create_string_buffer(2 * len(buf))
    parts = buf.raw.split(b"\0")[: 2 * n.value]
    return {parts[i].decode(): parts[i + 1].decode() for i in range(0, len(parts), 2)}


def save_prompt_cache(path: str, caches, metadata=None, stream=None):
    """savePromptCache(url:cache:metadata:) (KVCache.swift:1620-1680)."""
    hs = (C.c_void_p * max(1, len(caches)))(*[c._h.value for c in caches])
    keys, vals, n = _meta_args(metadata)
    _chk(lib().vkv_prompt_cache_save(path.encode(), hs, len(caches), keys, vals, n,
                                     stream_ptr(stream)))


def load_prompt_cache(path: str, stream=None):
    """loadPromptCache(url:) (KVCache.swift:1687-1780) -> (caches, metadata)."""
    n = C.c_int32()
    sp = stream_ptr(stream)
    _chk(lib().vkv_prompt_cache_load(path.encode(), sp, None, 0, C.byref(n), None, C.c_int64(0),
                                     None))
    count = C.c_int32()
    meta = _meta_out(lambda buf, ln, nm: _chk(lib().vkv_prompt_cache_load(
        path.encode(), sp, None, 0, C.byref(count), buf, ln, nm)))
    hs = (C.c_void_p * max(1, n.value))()
    _chk(lib().vkv_prompt_cache_load(path.encode(), sp, hs, n.value, C.byref(n), None,
                                     C.c_int64(0), None))
    return [_wrap_handle(C.c_void_p(hs[i])) for i in range(n.value)], meta


def save_prompt_cache_paged(path: str, pool, blocks, n_tokens: int, metadata=None, stream=None):
    """savePromptCache's file from one sequence's pool blocks (host ids)."""
    b = (C.c_int32 * max(1, len(blocks)))(*blocks)
    keys, vals, n = _meta_args(metadata)
    _chk(lib().vkv_prompt_cache_save_paged(path.encode(), pool._h, b, len(blocks),
                                           C.c_int64(n_tokens), keys, vals, n,
                                           stream_ptr(stream)))


def load_prompt_cache_paged(path: str, pool, blocks, stream=None):
    """A prompt-cache file into one sequence's pool blocks -> (n_tokens, metadata)."""
    b = (C.c_int32 * max(1, len(blocks)))(*blocks)
    nt = C.c_int64()

    def call(buf, ln, nm):
        _chk(lib().vkv_prompt_cache_load_paged(path.encode(), pool._h, b, len(blocks),
                                               C.byref(nt), buf, ln, nm, stream_ptr(stream)))

    meta = _meta_out(call)
    return nt.value, meta


def disk_hash_tokens(tokens, model_key=None, media_salt=None) -> str:
    """DiskCache.hashTokens (Cache/DiskCache.swift:659-682)."""
    t = (C.c_int64 * max(1, len(tokens)))(*tokens)
    out = C.create_string_buffer(33)
    _chk(lib().vkv_disk_hash_tokens(t, len(tokens),
                                    model_key.encode() if model_key is not None else None,
                                    media_salt.encode() if media_salt is not None else None, out))
    return out.value.decode()


def disk_cache_save(path: str, caches, stream=None):
    """TQDiskSerializer.serialize, format version 2."""
    hs = (C.c_void_p * max(1, len(caches)))(*[c._h.value for c in caches])
    _chk(lib().vkv_disk_cache_save(path.encode(), hs, len(caches), stream_ptr(stream)))


def disk_cache_load(path: str, stream=None):
    """TQDiskSerializer.deserializeV2 -> caches (None for a skipped layer)."""
    n = C.c_int32()
    _chk(lib().vkv_disk_cache_load(path.encode(), stream_ptr(stream), None, 0, C.byref(n)))
    hs = (C.c_void_p * max(1, n.value))()
    _chk(lib().vkv_disk_cache_load(path.encode(), stream_ptr(stream), hs, n.value, C.byref(n)))
    return [None if not hs[i] else _wrap_handle(C.c_void_p(hs[i])) for i in range(n.value)]
