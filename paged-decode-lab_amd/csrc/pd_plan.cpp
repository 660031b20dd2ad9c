// Host-only parts of the C ABI: error reporting, the split-KV planner and the
// metadata content check.  No HIP calls in this file.
#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>

#include "pd_internal.h"

namespace pd {

namespace {
thread_local char g_error[512] = "";
}

int fail(int status, const char* fmt, ...) {
  va_list args;
  va_start(args, fmt);
  std::vsnprintf(g_error, sizeof(g_error), fmt, args);
  va_end(args);
  return status;
}

void clear_error() { g_error[0] = '\0'; }

}  // namespace pd

extern "C" const char* pd_last_error(void) { return pd::g_error; }

extern "C" int pd_abi_version(void) { return PD_ABI_VERSION; }

namespace {

// Python's _f32 (splitkv_plan.py:11-12): round a double to the nearest float.
inline double f32(double x) { return static_cast<double>(static_cast<float>(x)); }

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

}  // namespace

// make_splitkv_plan (splitkv_plan.py:26-56).  The reference evaluates its
// heuristic in Python doubles and rounds to float32 at three points; each
// rounding below sits at the same place, and the .85*best comparison stays in
// double, so the chosen split count is bit-for-bit the reference's.
extern "C" int pd_make_plan(int32_t max_batch, int32_t num_heads, int32_t num_kv_heads,
                            int32_t head_dim, int32_t max_context_len, int32_t sm_count,
                            int32_t num_splits, pd_plan* out) {
  pd::clear_error();
  if (out == nullptr) return pd::fail(PD_EINVAL, "pd_make_plan: null output plan");
  if (max_batch <= 0 || num_heads <= 0 || num_kv_heads <= 0 || max_context_len <= 0)
    return pd::fail(PD_EINVAL, "batch, heads and context limits must be positive integers");
  if (!pd::valid_head_dim(head_dim))
    return pd::fail(PD_EINVAL, "custom decode supports head_dim 64, 128, or 256");
  if (num_heads % num_kv_heads)
    return pd::fail(PD_EINVAL, "query heads must be divisible by KV heads");
  if (sm_count < 1) return pd::fail(PD_EINVAL, "positive SM count required");
  if (num_splits < 0 || num_splits > 128)
    return pd::fail(PD_EINVAL, "num_splits must be an integer in [0,128]");
  if (num_heads / num_kv_heads > 16)
    return pd::fail(PD_EINVAL,
                    "matched split-KV requires at most 16 query heads per KV head");

  const int64_t tile = head_dim == 64 ? 256 : (head_dim == 128 ? 128 : 64);
  const int64_t width = ceil_div(max_context_len, pd::kPageSize);
  const int64_t capacity = width * 256;
  const int64_t blocks = ceil_div(capacity, tile);
  int64_t splits = num_splits;
  if (splits == 0) {
    const int64_t work = int64_t(max_batch) * num_kv_heads;
    const int64_t vsm = int64_t(sm_count) * 2;
    if (double(work) >= f32(f32(0.8) * double(vsm))) {
      splits = 1;
    } else {
      const int64_t top = std::min<int64_t>(std::min<int64_t>(128, vsm), blocks);
      double eff[129];
      bool eligible[129];
      double best = -1.0;
      for (int64_t n = 1; n <= top; ++n) {
        eligible[n] = n == 1 || ceil_div(blocks, n) != ceil_div(blocks, n - 1);
        if (!eligible[n]) continue;
        const double waves = f32(f32(double(work * n)) / double(vsm));
        eff[n] = f32(waves / std::ceil(waves));
        if (eff[n] > best) best = eff[n];
      }
      splits = 0;
      for (int64_t n = 1; n <= top && splits == 0; ++n)
        if (eligible[n] && eff[n] >= 0.85 * best) splits = n;
    }
  }
  int64_t padded = 1;
  while (padded < splits) padded <<= 1;
  const int64_t merge_rows = head_dim % 128 == 0 ? 4 : 8;
  out->splits = int32_t(splits);
  out->tile_tokens = int32_t(tile);
  out->tokens_per_split = int32_t(ceil_div(blocks, splits) * tile);
  out->table_capacity_tokens = int32_t(capacity);
  out->lse_lanes = int32_t(std::min<int64_t>(padded, 128 / merge_rows));
  out->sm_count = sm_count;
  out->is_explicit = num_splits ? 1 : 0;
  return PD_OK;
}

// Small-batch split of the base and fixed-split protocols.  The walks of
// pd_base / pd_split_fixed run one workgroup per (kv head group, sequence),
// and one workgroup streams about 76 GB/s, so a batch with fewer walks than
// half the CUs leaves most of the device idle.  Such a batch is cut into
// `chunks` partitions of `chunk_tokens` tokens (a multiple of 16384 / head_dim)
// per sequence, about sm_count / walks of them, at most 128 and at most one
// per 16384 / head_dim tokens of the table width: run through pd_split_fixed
// (one workgroup per partition) and merged by pd_ml_merge.  The walks are
// counted for the batch rounded up to a power of two, so that a batch padded
// up to a graph bucket of the same power of two gets the same plan.
extern "C" int pd_plan_chunks(int32_t batch, int32_t num_heads, int32_t num_kv_heads,
                              int32_t head_dim, int32_t table_width, int32_t sm_count,
                              int32_t* chunks, int32_t* chunk_tokens) {
  pd::clear_error();
  if (chunks == nullptr || chunk_tokens == nullptr)
    return pd::fail(PD_EINVAL, "pd_plan_chunks: null output");
  if (batch <= 0 || num_heads <= 0 || num_kv_heads <= 0)
    return pd::fail(PD_EINVAL, "batch and head counts must be positive");
  if (!pd::valid_head_dim(head_dim))
    return pd::fail(PD_EINVAL, "custom decode supports head_dim 64, 128, or 256");
  if (num_heads % num_kv_heads)
    return pd::fail(PD_EINVAL, "query heads must be divisible by KV heads");
  if (table_width < 1 || table_width >= (1 << 22))
    return pd::fail(PD_EINVAL, "table width must be in [1, 2^22)");
  if (sm_count < 1) return pd::fail(PD_EINVAL, "positive SM count required");
  int64_t rounded = 1;
  while (rounded < batch) rounded <<= 1;
  const int64_t walks = rounded * pd::walk_grid_y(num_heads, num_kv_heads, head_dim);
  const int64_t tile = 16384 / head_dim;
  const int64_t tiles = ceil_div(int64_t(table_width) * pd::kPageSize, tile);
  const int64_t want = std::min<int64_t>(std::min<int64_t>(sm_count / walks, 128), tiles);
  if (want < 2) {
    *chunks = 1;
    *chunk_tokens = int32_t(int64_t(table_width) * pd::kPageSize);
    return PD_OK;
  }
  const int64_t per = ceil_div(tiles, want);
  *chunks = int32_t(ceil_div(tiles, per));
  *chunk_tokens = int32_t(per * tile);
  return PD_OK;
}

// Bound on batch * num_heads * chunks over every batch <= max_batch and every
// table width: pd_plan_chunks never returns more than sm_count / walks chunks.
extern "C" int pd_chunk_rows(int32_t max_batch, int32_t num_heads, int32_t num_kv_heads,
                             int32_t head_dim, int32_t sm_count, int64_t* rows) {
  pd::clear_error();
  if (rows == nullptr) return pd::fail(PD_EINVAL, "pd_chunk_rows: null output");
  if (max_batch <= 0 || num_heads <= 0 || num_kv_heads <= 0)
    return pd::fail(PD_EINVAL, "batch and head counts must be positive");
  if (!pd::valid_head_dim(head_dim))
    return pd::fail(PD_EINVAL, "custom decode supports head_dim 64, 128, or 256");
  if (num_heads % num_kv_heads)
    return pd::fail(PD_EINVAL, "query heads must be divisible by KV heads");
  if (sm_count < 1) return pd::fail(PD_EINVAL, "positive SM count required");
  const int64_t y = pd::walk_grid_y(num_heads, num_kv_heads, head_dim);
  int64_t best = 0;
  for (int64_t b = 1; b <= max_batch && b * y * 2 <= sm_count; ++b) {
    const int64_t chunks = std::min<int64_t>(sm_count / (b * y), 128);
    best = std::max(best, b * num_heads * chunks);
  }
  *rows = best;
  return PD_OK;
}

// validate_metadata (reference.py:10-21) on host copies of table and lengths.
extern "C" int pd_validate_metadata(const int32_t* table, int64_t table_stride_b, int32_t width,
                                    const int32_t* lengths, int32_t batch, int64_t num_pages,
                                    int32_t max_context_len) {
  pd::clear_error();
  if (batch < 0 || width < 0 || (batch > 0 && (table == nullptr || lengths == nullptr)))
    return pd::fail(PD_EINVAL, "metadata batch dimensions differ");
  for (int32_t b = 0; b < batch; ++b) {
    const int64_t length = lengths[b];
    if (length < 0 || length > max_context_len)
      return pd::fail(PD_EINVAL, "context length outside configured capacity (row %d: %lld)", b,
                      static_cast<long long>(length));
    const int64_t live = ceil_div(length, pd::kPageSize);
    if (live > width) return pd::fail(PD_EINVAL, "invalid live page mapping (row %d)", b);
    const int32_t* row = table + int64_t(b) * table_stride_b;
    for (int64_t i = 0; i < live; ++i)
      if (row[i] < 0 || row[i] >= num_pages)
        return pd::fail(PD_EINVAL, "invalid live page mapping (row %d, entry %lld = %d)", b,
                        static_cast<long long>(i), row[i]);
  }
  return PD_OK;
}
