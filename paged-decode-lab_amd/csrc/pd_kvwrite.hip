// KV-cache writes into 256-slot NHD pages for MI355X (gfx950): the step
// before the decode path.  Byte copies, HBM-bound: every thread moves one
// 16-byte piece of a K row and the same piece of the V row with vector loads
// and stores; rows whose destination is negative are skipped.
//
//   pd_store_kv        token rows -> slots of a flat slot mapping
//                      (nano-vLLM store_kvcache, overlays/nano-vllm/nanovllm/
//                      layers/attention.py:10-38)
//   pd_store_kv_pages  [B, Hkv, S, D] chunks -> table[b, pos // 256] pages
//                      (PagedHybridCache.update, src/paged_decode/hybrid.py:63-72)
#include <hip/hip_runtime.h>

#include <cstdint>

#include "pd_internal.h"

namespace {

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;

// One 16-byte piece per thread: row = piece / kPieces, chunk = piece % kPieces.
// src rows are `src_stride` elements apart; dst row r goes to slot slots[r]
// (row_elems elements per slot).  A negative slot skips the row.
__global__ void __launch_bounds__(kThreads)
store_slots_kernel(const uint16_t* __restrict__ key, int64_t key_stride,
                   const uint16_t* __restrict__ value, int64_t value_stride,
                   uint16_t* __restrict__ k_cache, uint16_t* __restrict__ v_cache,
                   const int32_t* __restrict__ slots, int64_t rows, int pieces_per_row,
                   int64_t row_elems) {
  const int64_t piece = int64_t(blockIdx.x) * kThreads + threadIdx.x;
  if (piece >= rows * pieces_per_row) return;
  const int64_t r = piece / pieces_per_row;
  const int c = int(piece - r * pieces_per_row);
  const int32_t slot = slots[r];
  if (slot < 0) return;
  const int64_t dst = int64_t(slot) * row_elems + 8 * c;
  const u32x4_t kx = *reinterpret_cast<const u32x4_t*>(key + r * key_stride + 8 * c);
  const u32x4_t vx = *reinterpret_cast<const u32x4_t*>(value + r * value_stride + 8 * c);
  *reinterpret_cast<u32x4_t*>(k_cache + dst) = kx;
  *reinterpret_cast<u32x4_t*>(v_cache + dst) = vx;
}

// key[b, h, s, :] (strides ksb, ksh, kss; d contiguous) goes to the page slot
// table[b, pos[s] / 256] * 256 + pos[s] % 256, kv head h.  A negative
// position, a page index at or past the row's width, or a table entry outside
// [0, num_pages) skips it, so no row is written outside the page pool.
__global__ void __launch_bounds__(kThreads)
store_pages_kernel(const uint16_t* __restrict__ key, int64_t ksb, int64_t ksh, int64_t kss,
                   const uint16_t* __restrict__ value, int64_t vsb, int64_t vsh, int64_t vss,
                   uint16_t* __restrict__ k_pages, uint16_t* __restrict__ v_pages,
                   int64_t num_pages, const int32_t* __restrict__ table, int64_t tsb, int width,
                   const int64_t* __restrict__ positions, int batch, int hkv, int steps,
                   int pieces_per_row) {
  const int64_t piece = int64_t(blockIdx.x) * kThreads + threadIdx.x;
  const int64_t rows = int64_t(batch) * steps * hkv;
  if (piece >= rows * pieces_per_row) return;
  int64_t r = piece / pieces_per_row;
  const int c = int(piece - r * pieces_per_row);
  const int h = int(r % hkv);
  r /= hkv;
  const int s = int(r % steps);
  const int b = int(r / steps);
  const int64_t pos = positions[s];
  if (pos < 0 || (pos >> 8) >= width) return;
  const int32_t page = table[int64_t(b) * tsb + (pos >> 8)];
  if (page < 0 || page >= num_pages) return;
  const int D = pieces_per_row * 8;
  const int64_t dst = ((int64_t(page) * 256 + (pos & 255)) * hkv + h) * D + 8 * c;
  const u32x4_t kx = *reinterpret_cast<const u32x4_t*>(key + b * ksb + h * ksh + s * kss + 8 * c);
  const u32x4_t vx =
      *reinterpret_cast<const u32x4_t*>(value + b * vsb + h * vsh + s * vss + 8 * c);
  *reinterpret_cast<u32x4_t*>(k_pages + dst) = kx;
  *reinterpret_cast<u32x4_t*>(v_pages + dst) = vx;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

int launch_status(const char* what) {
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess)
    return pd::fail(PD_ELAUNCH, "%s launch failed: %s", what, hipGetErrorString(err));
  return PD_OK;
}

}  // namespace

extern "C" int pd_store_kv(const void* key, int64_t key_stride, const void* value,
                           int64_t value_stride, void* k_cache, void* v_cache,
                           const int32_t* slot_mapping, int64_t num_tokens, int32_t row_elems,
                           pd_stream_t stream) {
  pd::clear_error();
  if (num_tokens < 0) return pd::fail(PD_EINVAL, "num_tokens must be non-negative");
  if (num_tokens == 0) return PD_OK;
  if (!key || !value || !k_cache || !v_cache || !slot_mapping)
    return pd::fail(PD_EINVAL, "null tensor pointer");
  if (row_elems <= 0 || row_elems % 8)
    return pd::fail(PD_EINVAL, "num_kv_heads * head_dim must be a positive multiple of 8");
  if (!aligned16(key) || !aligned16(value) || !aligned16(k_cache) || !aligned16(v_cache) ||
      key_stride % 8 || value_stride % 8 || key_stride < row_elems || value_stride < row_elems)
    return pd::fail(PD_EINVAL,
                    "key/value rows and caches must be 16-byte aligned with strides of at least "
                    "num_kv_heads * head_dim elements, multiples of 8");
  const int pieces = row_elems / 8;
  const int64_t total = num_tokens * pieces;
  const int64_t blocks = (total + kThreads - 1) / kThreads;
  if (blocks > 0x7fffffff) return pd::fail(PD_EINVAL, "grid dimension exceeds device limits");
  hipLaunchKernelGGL(store_slots_kernel, dim3(unsigned(blocks)), dim3(kThreads), 0,
                     reinterpret_cast<hipStream_t>(stream), static_cast<const uint16_t*>(key),
                     key_stride, static_cast<const uint16_t*>(value), value_stride,
                     static_cast<uint16_t*>(k_cache), static_cast<uint16_t*>(v_cache),
                     slot_mapping, num_tokens, pieces, int64_t(row_elems));
  return launch_status("pd_store_kv");
}

extern "C" int pd_store_kv_pages(const void* key, int64_t key_stride_b, int64_t key_stride_h,
                                 int64_t key_stride_s, const void* value, int64_t value_stride_b,
                                 int64_t value_stride_h, int64_t value_stride_s, void* k_pages,
                                 void* v_pages, int64_t num_pages, const int32_t* table,
                                 int64_t table_stride_b,
                                 int32_t table_width, const int64_t* positions, int32_t batch,
                                 int32_t num_kv_heads, int32_t steps, int32_t head_dim,
                                 pd_stream_t stream) {
  pd::clear_error();
  if (batch <= 0 || num_kv_heads <= 0 || steps < 0)
    return pd::fail(PD_EINVAL, "batch and heads must be positive");
  if (steps == 0) return PD_OK;
  if (!pd::valid_head_dim(head_dim))
    return pd::fail(PD_EINVAL, "custom decode supports head_dim 64, 128, or 256");
  if (!key || !value || !k_pages || !v_pages || !table || !positions)
    return pd::fail(PD_EINVAL, "null tensor pointer");
  if (table_width < 1) return pd::fail(PD_EINVAL, "table width must be positive");
  if (num_pages < 1) return pd::fail(PD_EINVAL, "the page pool must hold at least one page");
  const int64_t strides[6] = {key_stride_b, key_stride_h, key_stride_s,
                              value_stride_b, value_stride_h, value_stride_s};
  for (int64_t st : strides)
    if (st % 8 || st < 0)
      return pd::fail(PD_EINVAL, "key/value strides must be non-negative multiples of 8");
  if (!aligned16(key) || !aligned16(value) || !aligned16(k_pages) || !aligned16(v_pages))
    return pd::fail(PD_EINVAL, "key/value and pages must be 16-byte aligned");
  const int pieces = head_dim / 8;
  const int64_t total = int64_t(batch) * steps * num_kv_heads * pieces;
  const int64_t blocks = (total + kThreads - 1) / kThreads;
  if (blocks > 0x7fffffff) return pd::fail(PD_EINVAL, "grid dimension exceeds device limits");
  hipLaunchKernelGGL(store_pages_kernel, dim3(unsigned(blocks)), dim3(kThreads), 0,
                     reinterpret_cast<hipStream_t>(stream), static_cast<const uint16_t*>(key),
                     key_stride_b, key_stride_h, key_stride_s, static_cast<const uint16_t*>(value),
                     value_stride_b, value_stride_h, value_stride_s,
                     static_cast<uint16_t*>(k_pages), static_cast<uint16_t*>(v_pages), num_pages,
                     table, table_stride_b, table_width, positions, batch, num_kv_heads, steps,
                     pieces);
  return launch_status("pd_store_kv_pages");
}
