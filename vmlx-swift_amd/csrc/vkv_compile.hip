// vkv_compile.hip -- device-offset operations behind the fixed-buffer
// caches (CompilableKVCache, CompilableRotatingKVCache):
//
//   * dynamic slice / slice update: a copy whose start along one axis is an
//     int32 read from device memory by the kernel itself
//     (dynamicSlice / dynamicSliceUpdate, MLXLMCommon/DynamicSlice.swift:
//     21-71 -> mlx_slice_dynamic / mlx_slice_update_dynamic);
//   * the write counters (offset, ring index) advanced on the device
//     (CompilableKVCache.swift:117-148, CompilableRotatingKVCache.swift:
//     157-207);
//   * the full-buffer attention mask computed from the device offset
//     (CompilableKVCache.swift:167-193, CompilableRotatingKVCache.swift:
//     233-260);
//   * the host-offset masks: createCausalMask, the rotating cache's rolled
//     row and the batch mask of createBatchCausalMask
//     (BatchEngine/BatchMask.swift:44-115).
//
// No host read of the offset is needed between steps, so a decode step
// built from these launches can be captured once in a HIP graph and
// replayed (the HIP counterpart of the reference's compile()).  The start
// is clamped so that the copied block stays inside the array, as XLA's
// dynamic_update_slice does; in-range starts give the reference's result.
#include <algorithm>

#include "vkv_device.h"
#include "vkv_internal.h"

namespace vkv {

namespace {

template <int ES>
struct Elem;
template <>
struct Elem<1> {
  using T = uint8_t;
};
template <>
struct Elem<2> {
  using T = uint16_t;
};
template <>
struct Elem<4> {
  using T = uint32_t;
};

// One thread per element of the copied block (row-major over shape).
template <int ES>
__global__ void __launch_bounds__(256) dyn_copy_kernel(DynCopy c) {
  using T = typename Elem<ES>::T;
  const int64_t n = c.shape[0] * c.shape[1] * c.shape[2] * c.shape[3];
  const int64_t lo = 0, hi = c.limit - c.shape[c.axis];
  int64_t s = *c.start;
  s = s < lo ? lo : (s > hi ? hi : s);
  for (int64_t e = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; e < n;
       e += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    int64_t i[4];
    int64_t r = e;
    i[3] = r % c.shape[3];
    r /= c.shape[3];
    i[2] = r % c.shape[2];
    r /= c.shape[2];
    i[1] = r % c.shape[1];
    i[0] = r / c.shape[1];
    int64_t so = 0, dof = 0;
#pragma unroll
    for (int d = 0; d < 4; d++) {
      const int64_t off = (d == c.axis) ? s : 0;
      so += (i[d] + (c.on_dst ? 0 : off)) * c.sstr[d];
      dof += (i[d] + (c.on_dst ? off : 0)) * c.dstr[d];
    }
    reinterpret_cast<T*>(c.dst)[dof] = reinterpret_cast<const T*>(c.src)[so];
  }
}

// ctr[0] += n; ring caches also advance ctr[1] with the reference's wrap
// (CompilableRotatingKVCache.swift:178-193).
__global__ void counter_advance_kernel(int32_t* ctr, int32_t n, int32_t ring, int32_t max_size,
                                       int32_t keep) {
  if (threadIdx.x != 0 || blockIdx.x != 0) return;
  ctr[0] += n;
  if (ring) {
    const int32_t adv = ctr[1] + n;
    int32_t rot;
    if (keep > 0)
      rot = keep + (adv - keep) % (max_size - keep);
    else
      rot = adv % max_size;
    ctr[1] = adv < max_size ? adv : rot;
  }
}

__global__ void counter_advance_both_kernel(int32_t* ctr, int32_t n) {
  if (threadIdx.x == 0 && blockIdx.x == 0) {
    ctr[0] += n;
    ctr[1] += n;
  }
}

__global__ void counter_set_kernel(int32_t* ctr, int32_t offset, int32_t idx) {
  if (threadIdx.x == 0 && blockIdx.x == 0) {
    ctr[0] = offset;
    ctr[1] = idx;
  }
}

// mask[i][j] = j <= off + i (and, on a ring that has wrapped, all true),
// then & j >= off + i - (window - 1) when a window is given.
__global__ void __launch_bounds__(256) offset_mask_kernel(const int32_t* ctr, int32_t n,
                                                          int32_t cols, int32_t window,
                                                          int32_t ring, uint8_t* mask) {
  const int64_t off = ctr[0];
  const int64_t total = static_cast<int64_t>(n) * cols;
  for (int64_t e = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; e < total;
       e += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t i = e / cols, j = e % cols;
    const int64_t l = off + i;
    bool m = l >= j;
    if (ring && l >= cols) m = true;
    if (window > 0) m = m && (j >= l - (window - 1));
    mask[e] = m;
  }
}

// createCausalMask (KVCache.swift:314-336) with a host offset: [n, off + n]
// bool, row i (the query at off + i) sees key j when off + i >= j and, with
// a window, off + i < j + window.
__global__ void __launch_bounds__(256) causal_mask_kernel(int32_t n, int64_t off, int32_t window,
                                                          uint8_t* mask) {
  const int64_t cols = off + n, total = static_cast<int64_t>(n) * cols;
  for (int64_t e = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; e < total;
       e += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t i = e / cols, j = e % cols;
    bool m = off + i >= j;
    if (window > 0) m = m && (off + i < j + window);
    mask[e] = m;
  }
}

// The rotating cache's single-token window mask (KVCache.swift:905-923):
// roll(arange(size) >= size - window, shift) -- element j holds the base
// element (j - shift) mod size.
__global__ void __launch_bounds__(256) roll_mask_kernel(int64_t size, int64_t window,
                                                        int64_t shift, uint8_t* mask) {
  for (int64_t j = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; j < size;
       j += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t i = ((j - shift) % size + size) % size;
    mask[j] = i >= size - window;
  }
}

// createBatchCausalMask (BatchEngine/BatchMask.swift:44-115) for up to
// kBatchMaskSlots slots per launch: mask [B, 1, n, cols] as bytes, slot b
// row i column j.  A slot whose key length is below offset + n has wrapped
// its ring: every key below the key length is visible.  Otherwise key j is
// visible to the query at l = offset + i when j <= l, j < keyLen and, with
// a window (window >= 0), j >= l - (window - 1).  Each thread writes 16
// consecutive bytes of the launch's range [slot0 * n * cols, slot1 * n *
// cols) with one vector store when they are aligned and in range.
struct BatchMaskArgs {
  int32_t n, cols, window, slot0, slots;
  int32_t offset[kBatchMaskSlots];
  int32_t key_len[kBatchMaskSlots];
};

__global__ void __launch_bounds__(256) batch_mask_kernel(BatchMaskArgs a, uint8_t* mask) {
  const int64_t row = static_cast<int64_t>(a.n) * a.cols;
  const int64_t lo = a.slot0 * row, hi = (a.slot0 + static_cast<int64_t>(a.slots)) * row;
  const int64_t first = lo & ~static_cast<int64_t>(15);
  for (int64_t c = first + (static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x) * 16;
       c < hi; c += static_cast<int64_t>(gridDim.x) * blockDim.x * 16) {
    uint32_t w[4] = {0, 0, 0, 0};
    const int64_t e0 = c < lo ? lo : c;
    int64_t b = e0 / row, r = e0 - b * row;
    int64_t i = r / a.cols, j = r - i * a.cols;
    for (int t = static_cast<int>(e0 - c); t < 16 && c + t < hi; ++t) {
      const int64_t off = a.offset[b - a.slot0], kl = a.key_len[b - a.slot0];
      bool m;
      if (kl < off + a.n) {
        m = j < kl;
      } else {
        const int64_t l = off + i;
        m = l >= j && j < kl;
        if (a.window >= 0) m = m && j >= l - (a.window - 1);
      }
      w[t >> 2] |= static_cast<uint32_t>(m) << (8 * (t & 3));
      if (++j == a.cols) {
        j = 0;
        if (++i == a.n) {
          i = 0;
          ++b;
        }
      }
    }
    if (c >= lo && c + 16 <= hi) {
      *reinterpret_cast<uint4*>(mask + c) = make_uint4(w[0], w[1], w[2], w[3]);
    } else {
      for (int t = 0; t < 16; ++t)
        if (c + t >= lo && c + t < hi) mask[c + t] = static_cast<uint8_t>(w[t >> 2] >> (8 * (t & 3)));
    }
  }
}

int blocks_for(int64_t n) {
  return static_cast<int>(std::min<int64_t>((n + 255) / 256, 4096));
}

}  // namespace

void launch_dyn_copy(int esize, const DynCopy& c, hipStream_t st) {
  const int64_t n = c.shape[0] * c.shape[1] * c.shape[2] * c.shape[3];
  if (n <= 0) return;
  VKV_CHECK(c.axis >= 0 && c.axis < 4, "axis out of range");
  VKV_CHECK(c.shape[c.axis] <= c.limit, "the copied block is larger than the array along the axis");
  const int g = blocks_for(n);
  if (esize == 1)
    hipLaunchKernelGGL(dyn_copy_kernel<1>, dim3(g), dim3(256), 0, st, c);
  else if (esize == 2)
    hipLaunchKernelGGL(dyn_copy_kernel<2>, dim3(g), dim3(256), 0, st, c);
  else if (esize == 4)
    hipLaunchKernelGGL(dyn_copy_kernel<4>, dim3(g), dim3(256), 0, st, c);
  else
    throw Error("element size must be 1, 2 or 4 bytes");
  VKV_HIP(hipGetLastError());
}

void launch_counter_advance(int32_t* ctr, int n, int ring, int max_size, int keep, hipStream_t st) {
  hipLaunchKernelGGL(counter_advance_kernel, dim3(1), dim3(64), 0, st, ctr, n, ring, max_size, keep);
  VKV_HIP(hipGetLastError());
}

void launch_counter_advance_both(int32_t* ctr, int n, hipStream_t st) {
  hipLaunchKernelGGL(counter_advance_both_kernel, dim3(1), dim3(64), 0, st, ctr, n);
  VKV_HIP(hipGetLastError());
}

void launch_counter_set(int32_t* ctr, int32_t offset, int32_t idx, hipStream_t st) {
  hipLaunchKernelGGL(counter_set_kernel, dim3(1), dim3(64), 0, st, ctr, offset, idx);
  VKV_HIP(hipGetLastError());
}

void launch_offset_mask(const int32_t* ctr, int n, int cols, int window, int ring, uint8_t* mask,
                        hipStream_t st) {
  const int64_t total = static_cast<int64_t>(n) * cols;
  if (total <= 0) return;
  hipLaunchKernelGGL(offset_mask_kernel, dim3(blocks_for(total)), dim3(256), 0, st, ctr, n, cols,
                     window, ring, mask);
  VKV_HIP(hipGetLastError());
}

void launch_causal_mask(int n, int64_t off, int window, uint8_t* mask, hipStream_t st) {
  const int64_t total = static_cast<int64_t>(n) * (off + n);
  if (total <= 0) return;
  hipLaunchKernelGGL(causal_mask_kernel, dim3(blocks_for(total)), dim3(256), 0, st, n, off, window,
                     mask);
  VKV_HIP(hipGetLastError());
}

void launch_roll_mask(int64_t size, int64_t window, int64_t shift, uint8_t* mask, hipStream_t st) {
  if (size <= 0) return;
  hipLaunchKernelGGL(roll_mask_kernel, dim3(blocks_for(size)), dim3(256), 0, st, size, window,
                     shift, mask);
  VKV_HIP(hipGetLastError());
}

void launch_batch_mask(int n, int cols, int window, const int32_t* offsets, const int32_t* key_lens,
                       int batch, uint8_t* mask, hipStream_t st) {
  VKV_CHECK(reinterpret_cast<uintptr_t>(mask) % 16 == 0, "the batch mask must be 16-byte aligned");
  for (int s0 = 0; s0 < batch; s0 += kBatchMaskSlots) {
    BatchMaskArgs a{};
    a.n = n;
    a.cols = cols;
    a.window = window;
    a.slot0 = s0;
    a.slots = std::min(kBatchMaskSlots, batch - s0);
    for (int b = 0; b < a.slots; ++b) {
      a.offset[b] = offsets[s0 + b];
      a.key_len[b] = key_lens[s0 + b];
    }
    const int64_t bytes = static_cast<int64_t>(a.slots) * n * cols;
    if (bytes <= 0) continue;
    hipLaunchKernelGGL(batch_mask_kernel, dim3(blocks_for((bytes + 31) / 16)), dim3(256), 0, st, a,
                       mask);
    VKV_HIP(hipGetLastError());
  }
}

}  // namespace vkv
