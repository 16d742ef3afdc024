"""Test infrastructure only: numpy / pure-Python restatement of the
reference's cache state machines (the checker for the C++ caches).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use it.
Each class follows the cited Swift method line by line in behaviour; arrays
are numpy (bf16/f16 carried as uint16 bit patterns, which is exact for the
pure data movement these caches do).  Quantization goes through the C
oracle (oracle.py).

Pins: offsets/capacities/returned lengths follow closed-form index rules;
the tests also check the reference's own scenario expectations
(Tests/MLXLMTests/KVCacheTests.swift:15-141,
Tests/MLXLMCommonFocusedTests/RotatingKVCachePhysicalGrowthTests.swift:30-74,
Tests/MLXLMTests/PagedCacheTests.swift:8-186, CacheBlockTests.swift:284-329)
and invariants (temporal order of a ring equals the last tokens written).
"""
from __future__ import annotations

import hashlib
import struct
from typing import Optional

import numpy as np


def _cat(parts):
    parts = [p for p in parts if p is not None]
    return np.concatenate(parts, axis=2)


class KVCacheSimpleRef:
    """KVCache.swift:452-596."""

    def __init__(self, step: int = 256):
        self.step = step
        self.keys = None
        self.values = None
        self.offset = 0

    def update(self, keys, values):  # :465-508
        prev = self.offset
        S = keys.shape[2]
        reset = self.keys is None or prev + S > self.keys.shape[2]
        if reset:
            B, H, _, D = keys.shape
            Dv = values.shape[3]
            n = (self.step + S - 1) // self.step
            nk = np.zeros((B, H, n * self.step, D), keys.dtype)
            nv = np.zeros((B, H, n * self.step, Dv), values.dtype)
            if self.keys is not None:
                ck, cv = self.keys, self.values
                if prev % self.step != 0:
                    ck, cv = ck[:, :, :prev], cv[:, :, :prev]
                self.keys, self.values = _cat([ck, nk]), _cat([cv, nv])
            else:
                self.keys, self.values = nk, nv
        self.offset += S
        self.keys[:, :, prev:self.offset] = keys
        self.values[:, :, prev:self.offset] = values
        return self.keys[:, :, :self.offset], self.values[:, :, :self.offset]

    @property
    def state(self):
        if self.keys is None:
            return []
        return [self.keys[:, :, :self.offset], self.values[:, :, :self.offset]]

    def trim(self, n):
        t = min(self.offset, n)
        self.offset -= t
        return t


class RotatingKVCacheRef:
    """KVCache.swift:605-958."""

    def __init__(self, max_size: int, keep: int = 0, step: int = 256):
        self.max_size, self.keep, self.step = max_size, keep, step
        self.keys = self.values = None
        self.offset = 0
        self.idx = 0

    def _trim(self, trim_size, a, append=None):  # :626-640
        parts = [a[:, :, :self.keep], a[:, :, trim_size + self.keep:]] if trim_size > 0 else [a]
        if append is not None:
            parts.append(append)
        return _cat(parts)

    def _temporal_order(self, a):  # :642-656
        if self.idx == a.shape[2]:
            return a
        if self.idx < self.offset:
            return _cat([a[:, :, :self.keep], a[:, :, self.idx:], a[:, :, self.keep:self.idx]])
        return a[:, :, :self.idx]

    def _update_concat(self, k, v):  # :658-680
        if self.keys is None:
            self.keys, self.values = k.copy(), v.copy()
        else:
            self.keys = self._temporal_order(self.keys)
            self.values = self._temporal_order(self.values)
            self.idx = self.keys.shape[2]
            trim = self.idx - self.max_size + 1
            self.keys = self._trim(trim, self.keys, k)
            self.values = self._trim(trim, self.values, v)
        self.offset += k.shape[2]
        self.idx = self.keys.shape[2]
        return self.keys, self.values

    def _update_in_place(self, k, v):  # :682-769
        B, H, S, D = k.shape
        prev = self.offset
        fill = 0 if self.keys is None else self.keys.shape[2]
        if self.keys is None or (prev >= fill and fill < self.max_size):
            ns = min(self.step, self.max_size - fill)
            nk = np.zeros((B, H, ns, D), k.dtype)
            nv = np.zeros((B, H, ns, v.shape[3]), v.dtype)
            if self.keys is not None:
                self.keys, self.values = _cat([self.keys, nk]), _cat([self.values, nv])
            else:
                self.keys, self.values = nk, nv
            self.idx = fill
        trim = self.keys.shape[2] - self.max_size
        if trim > 0:
            self.keys = self._trim(trim, self.keys)
            self.values = self._trim(trim, self.values)
            self.idx = self.max_size
        if self.idx == self.max_size:
            self.idx = self.keep
        cap = self.keys.shape[2]
        if self.idx + S > cap:
            self.idx = self.keep
        if self.idx + S > cap:
            return self._update_concat(k, v)
        self.keys[:, :, self.idx:self.idx + S] = k
        self.values[:, :, self.idx:self.idx + S] = v
        self.offset += S
        self.idx += S
        if self.offset < self.max_size:
            return self.keys[:, :, :self.offset], self.values[:, :, :self.offset]
        return self.keys, self.values

    def _can_update_in_place(self, S):  # :780-789
        if self.keys is None:
            return True
        cap = self.keys.shape[2]
        grown = self.offset >= cap and cap < self.max_size
        eff = min(cap + self.step, self.max_size) if grown else cap
        start = self.keep if self.idx >= eff else self.idx
        return start + S <= eff

    def update(self, k, v):  # :791-799
        if k.shape[2] == 1 and self._can_update_in_place(1):
            return self._update_in_place(k, v)
        return self._update_concat(k, v)

    @property
    def state(self):
        if self.keys is None:
            return []
        if self.offset < self.keys.shape[2]:
            return [self.keys[:, :, :self.offset], self.values[:, :, :self.offset]]
        return [self.keys, self.values]

    @property
    def meta_state(self):
        return [str(self.keep), str(self.max_size), str(self.step), str(self.offset), str(self.idx)]

    def trim(self, n):
        t = min(self.offset, n)
        self.offset -= t
        self.idx -= t
        return t

    def temporally_ordered(self):  # :876-887
        k, v = self._temporal_order(self.keys), self._temporal_order(self.values)
        if self.offset < k.shape[2]:
            return k[:, :, :self.offset], v[:, :, :self.offset]
        return k, v

    def make_mask(self, n, window=None, return_array=False):  # :890-927
        if n > 1:
            actual = window if window is not None else self.max_size
            capped = min(self.max_size - 1, self.offset)
            if capped + n > actual or return_array:
                return causal_mask(n, capped, actual)
            return "causal"
        if window is None:
            return "none"
        if self.offset >= window and self.max_size > window:
            cur = self.idx if self.idx < self.max_size else 0
            size = self.offset + 1 if self.offset < self.max_size else self.max_size
            m = np.arange(size) >= size - window
            return np.roll(m, cur + 1)
        return "none"


def dynamic_slice_update_ref(dst, update, start, axis):
    """dynamicSliceUpdate (DynamicSlice.swift:50-71) on numpy arrays: a copy
    of dst with update written at `start` along axis.  Starts are clamped so
    the update fits (the XLA dynamic_update_slice rule; the reference only
    issues in-range starts)."""
    out = dst.copy()
    s = int(min(max(start, 0), dst.shape[axis] - update.shape[axis]))
    idx = [slice(None)] * dst.ndim
    idx[axis] = slice(s, s + update.shape[axis])
    out[tuple(idx)] = update
    return out


def dynamic_slice_ref(src, start, axis, size):
    """dynamicSlice (DynamicSlice.swift:21-48), clamped like the update."""
    s = int(min(max(start, 0), src.shape[axis] - size))
    idx = [slice(None)] * src.ndim
    idx[axis] = slice(s, s + size)
    return src[tuple(idx)].copy()


class CompilableKVCacheRef:
    """CompilableKVCache.swift:40-262: fixed [B, H, maxLength, D] buffers,
    update writes at offset and returns the whole buffers, makeMask is always
    an array mask over the buffer."""

    def __init__(self, max_length=4096, step=256):
        self.max_length, self.step = max_length, step
        self.keys = self.values = None
        self.offset = 0

    @classmethod
    def from_state(cls, state, max_length=4096):  # :62-86
        c = cls(max_length)
        if len(state) >= 2:
            c.state = state
        return c

    def update(self, k, v):  # :115-149
        if self.keys is None:
            B, H, _, D = k.shape
            self.keys = np.zeros((B, H, self.max_length, D), k.dtype)
            self.values = np.zeros((B, H, self.max_length, v.shape[3]), v.dtype)
        self.keys = dynamic_slice_update_ref(self.keys, k, self.offset, 2)
        self.values = dynamic_slice_update_ref(self.values, v, self.offset, 2)
        self.offset += k.shape[2]
        return self.keys, self.values

    def make_mask(self, n, window=None):  # :167-193
        linds = (self.offset + np.arange(n))[:, None]
        rinds = np.arange(self.max_length)[None]
        m = linds >= rinds
        if window is not None:
            m &= rinds >= linds - (window - 1)
        return m

    @property
    def state(self):  # :197-211
        if self.keys is None:
            return []
        if self.offset == self.keys.shape[2]:
            return [self.keys, self.values]
        return [self.keys[:, :, :self.offset], self.values[:, :, :self.offset]]

    @state.setter
    def state(self, arrays):  # :212-225
        k, v = arrays[0], arrays[1]
        L = k.shape[2]
        self.keys = np.zeros(k.shape[:2] + (self.max_length, k.shape[3]), k.dtype)
        self.values = np.zeros(v.shape[:2] + (self.max_length, v.shape[3]), v.dtype)
        self.keys[:, :, :L] = k
        self.values[:, :, :L] = v
        self.offset = L

    def trim(self, n):  # :229-240
        t = min(self.offset, n)
        self.offset -= t
        return t


class CompilableRotatingKVCacheRef:
    """BatchEngine/CompilableRotatingKVCache.swift:1-265, with the counters
    as plain ints (the reference keeps them in MLXArrays)."""

    def __init__(self, max_size, keep=0, step=256):
        self.max_size, self.keep, self.step = max_size, keep, step
        self.keys = self.values = None
        self.idx = 0
        self.offset = 0

    @classmethod
    def from_rotating(cls, r):  # :91-150
        c = cls(r.max_size, r.keep, r.step)
        c.idx, c.offset = r.idx, r.offset
        if r.keys is not None:
            cur = r.keys.shape[2]
            if cur < c.max_size:
                pad = c.max_size - cur
                B, H, _, D = r.keys.shape
                c.keys = _cat([r.keys, np.zeros((B, H, pad, D), r.keys.dtype)])
                c.values = _cat([r.values, np.zeros((B, H, pad, r.values.shape[3]), r.values.dtype)])
            else:
                c.keys, c.values = r.keys.copy(), r.values.copy()
        return c

    def update(self, k, v):  # :157-207
        if self.keys is None:
            B, H, _, D = k.shape
            self.keys = np.zeros((B, H, self.max_size, D), k.dtype)
            self.values = np.zeros((B, H, self.max_size, v.shape[3]), v.dtype)
        self.keys = dynamic_slice_update_ref(self.keys, k, self.idx, 2)
        self.values = dynamic_slice_update_ref(self.values, v, self.idx, 2)
        adv = self.idx + k.shape[2]
        if self.keep > 0:
            rot = self.keep + (adv - self.keep) % (self.max_size - self.keep)
        else:
            rot = adv % self.max_size
        self.idx = adv if adv < self.max_size else rot
        self.offset += k.shape[2]
        return self.keys, self.values

    def make_mask(self, n, window=None):  # :233-260
        linds = (self.offset + np.arange(n))[:, None]
        rinds = np.arange(self.max_size)[None]
        m = np.where(linds >= self.max_size, True, linds >= rinds)
        if window is not None:
            m &= rinds >= linds - (window - 1)
        return m


def causal_mask(n, offset, window=None):
    """createCausalMask (KVCache.swift:314-336)."""
    r = np.arange(offset + n)[None]
    l = np.arange(offset, offset + n)[:, None]
    m = l >= r
    if window is not None:
        m &= l < r + window
    return m


def batch_causal_mask(n, offsets, key_lens=None, window=None):
    """createBatchCausalMask (BatchEngine/BatchMask.swift:44-115): bool
    [B, 1, n, maxTotal]; a slot whose key length is below offset + n has
    wrapped and sees every key below its length (:80-94), otherwise the
    causal (+ window) test on positions offset + i, cut at the key length
    (:95-111)."""
    assert len(offsets) > 0
    kls = list(key_lens) if key_lens is not None else [o + n for o in offsets]
    total = max(kls)
    r = np.arange(total)[None]
    out = np.zeros((len(offsets), 1, n, total), bool)
    for b, (off, kl) in enumerate(zip(offsets, kls)):
        if kl < off + n:
            m = np.broadcast_to(r < kl, (n, total))
        else:
            l = (np.arange(n) + off)[:, None]
            m = l >= r
            if window is not None:
                m = m & (r >= l - (window - 1))
            m = m & (r < kl)
        out[b, 0] = m
    return out


def base_make_mask(offset, n, window=None, return_array=False):
    """BaseKVCache.makeMask (KVCache.swift:287-311)."""
    if n == 1:
        return "none"
    if offset > 0 or return_array or (window is not None and n > window):
        return causal_mask(n, offset, window)
    return "causal"


class QuantizedKVCacheRef:
    """KVCache.swift:961-1221 (storage capacities only; codes via oracle)."""

    def __init__(self, group_size=64, bits=8, step=256):
        self.group_size, self.bits, self.step = group_size, bits, step
        self.cap = 0
        self.offset = 0
        self.rows = None  # list of (wq, scales, biases) for keys / values, reference layout

    def update_quantized(self, keys, values, dtype):  # :1049-1122
        import oracle as O

        prev = self.offset
        S = keys.shape[2]
        if self.rows is None or prev + S > self.cap:
            new = ((self.step + S - 1) // self.step) * self.step
            if self.rows is not None:
                base = prev if prev % self.step != 0 else self.cap
                self.cap = base + new
            else:
                self.cap = new
        self.offset += S
        qk = O.quantize(keys, dtype, self.group_size, self.bits)[:3]
        qv = O.quantize(values, dtype, self.group_size, self.bits)[:3]
        if self.rows is None:
            self.rows = [list(qk), list(qv)]
            self._len = S
        else:
            for i in range(2):
                q = (qk, qv)[i]
                for j in range(3):
                    cur = self.rows[i][j][:, :, :prev]
                    self.rows[i][j] = np.concatenate([cur, q[j]], axis=2)
        return self.state

    @property
    def state(self):
        if self.rows is None:
            return []
        return [a[:, :, :self.offset] for i in range(2) for a in self.rows[i]]

    @property
    def meta_state(self):
        return [str(self.step), str(self.offset), str(self.group_size), str(self.bits)]


# ----------------------------------------------------------------- prefix
def block_hash(parent: Optional[str], tokens, model_key=None, media_salt=None) -> str:
    """CacheBlock.computeBlockHash (CacheBlock.swift:110-146) with hashlib."""
    h = hashlib.sha256()
    if model_key is not None:
        h.update(model_key.encode())
    if media_salt is not None:
        h.update(b"|media:")
        h.update(media_salt.encode())
    if parent is not None:
        h.update(parent.encode())
    h.update(b"".join(struct.pack("<q", t) for t in tokens))
    return h.hexdigest()


class _Blk:
    def __init__(self, bid):
        self.id = bid
        self.hash = None
        self.tokens = []
        self.data = False
        self.ref = 0


class PagedCacheManagerRef:
    """PagedCacheManager.swift:38-377 with FreeBlockQueue / BlockHashMap."""

    def __init__(self, block_size=64, max_blocks=1000, model_key=None):
        self.bs, self.maxb, self.key = block_size, max_blocks, model_key
        self.blocks = [_Blk(i) for i in range(max_blocks)]
        self.queue = list(range(1, max_blocks))  # LRU order, front = oldest
        self.map = {}
        self.stats = dict(total_blocks=max_blocks, allocated_blocks=0, free_blocks=max_blocks - 1,
                          cache_hits=0, cache_misses=0, evictions=0)

    def _reset(self, b):
        b.hash, b.tokens, b.data, b.ref = None, [], False, 0

    def allocate_block(self):  # :116-127
        if not self.queue:
            return None
        b = self.blocks[self.queue.pop(0)]
        if b.hash is not None:
            self.map.pop(b.hash, None)
            self.stats["evictions"] += 1
        self._reset(b)
        b.ref += 1
        self.stats["allocated_blocks"] += 1
        self.stats["free_blocks"] -= 1
        return b.id

    def free_block(self, bid):  # :142-156
        b = self.blocks[bid]
        was = b.ref > 0
        b.ref = max(0, b.ref - 1)
        if b.ref == 0:
            if b.hash is None or not b.data or not b.tokens:
                if b.hash is not None and self.map.get(b.hash) == bid:
                    del self.map[b.hash]
                self._reset(b)
            if bid not in self.queue:
                self.queue.append(bid)
            if was:
                self.stats["allocated_blocks"] -= 1
                self.stats["free_blocks"] += 1

    def writable(self, bid):
        """Copy-on-write before writing into block bid (the library's
        vkv_prefix_writable; no reference counterpart): the block itself
        when the caller holds the only reference and no cache entry names
        it, else a freshly allocated block (None if none is free) that
        takes over the caller's reference."""
        b = self.blocks[bid]
        assert b.ref >= 1
        if b.ref == 1 and b.hash is None:
            return bid
        nb = self.allocate_block()
        if nb is None:
            return None
        self.free_block(bid)
        return nb

    def _pin(self, b):
        if b.ref == 0 and b.id in self.queue:
            self.queue.remove(b.id)
            self.stats["allocated_blocks"] += 1
            self.stats["free_blocks"] -= 1
        b.ref += 1

    def store_token_sequence(self, tokens, n_data_chunks, media_salt=None):  # :229-310
        pinned, parent, ci, off = [], None, 0, 0
        while off < len(tokens):
            end = min(off + self.bs, len(tokens))
            chunk = list(tokens[off:end])
            h = block_hash(parent, chunk, self.key, media_salt)
            if h in self.map:
                ex = self.blocks[self.map[h]]
                self._pin(ex)
                pinned.append(ex.id)
                parent, off, ci = h, end, ci + 1
                continue
            if ci >= n_data_chunks:
                break
            bid = self.allocate_block()
            if bid is None:
                break
            b = self.blocks[bid]
            b.tokens, b.data, b.hash = chunk, True, h
            self.map[h] = bid
            pinned.append(bid)
            parent, off, ci = h, end, ci + 1
        for bid in reversed(pinned):
            self.free_block(bid)

    def _partial(self, parent, chunk, media_salt):  # BlockHashMap.swift:42-70
        best = None
        for bid in self.map.values():
            b = self.blocks[bid]
            st = b.tokens
            if not st or len(st) >= self.bs or len(st) >= len(chunk) or chunk[:len(st)] != st:
                continue
            if b.hash != block_hash(parent, st, self.key, media_salt):
                continue
            if best is None or len(st) > len(best.tokens) or (
                    len(st) == len(best.tokens) and b.id < best.id):
                best = b
        return best

    def fetch_prefix(self, tokens, media_salt=None):  # :320-376
        parent, got, off = None, [], 0
        while off < len(tokens):
            end = min(off + self.bs, len(tokens))
            chunk = list(tokens[off:end])
            h = block_hash(parent, chunk, self.key, media_salt)
            exact = h in self.map
            b = self.blocks[self.map[h]] if exact else self._partial(parent, chunk, media_salt)
            if b is None:
                self.stats["cache_misses"] += 1
                break
            self.stats["cache_hits"] += 1
            self._pin(b)
            got.append(b.id)
            parent = b.hash
            off += len(b.tokens)
            if not exact:
                break
        if not got:
            return None
        m = sum(len(self.blocks[i].tokens) for i in got)
        return m, list(tokens[off:]), got
