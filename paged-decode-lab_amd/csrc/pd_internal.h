// Internal helpers shared by the host sources of libpaged_decode.so.
#pragma once

#include <cstdarg>
#include <cstdint>

#include "paged_decode.h"

namespace pd {

// Records a printf-style message for pd_last_error() and returns `status`.
int fail(int status, const char* fmt, ...) __attribute__((format(printf, 2, 3)));

// Clears the calling thread's error message.
void clear_error();

constexpr int kPageSize = PD_PAGE_SIZE;
constexpr int kPartitionSize = PD_PARTITION_SIZE;

inline bool valid_head_dim(int d) { return d == 64 || d == 128 || d == 256; }

// kv heads per workgroup of the D = 64 base / fixed-split launch: 4 when the
// kv head count is a multiple of 4 and the four heads' query heads fit one
// 16-head group, else 2 when it is even and a pair's do, else 1.  A token's
// rows of the workgroup's heads are then one contiguous run of 128 bytes per
// head (512 bytes for four).  With the loader kernel, four heads beat pairs by
// 5-7% (batch 128, 16 kv heads, lengths up to 4096: 157.6 against 165.7 us
// base, 162.1 against 174.2 us fixed split); eight heads (32-token tiles)
// took 262 us: the longest sequences' workgroups then set the call.  (Pairs
// at D = 128, whose rows are 256 bytes already, lost 3-17% with 8 kv heads in
// the kernel before the loader wavefronts: 979 against 814 us for batch 64,
// Hq 32, Hkv 8, lengths up to 32768.)
inline int heads_per_workgroup(int num_kv_heads, int G) {
  if (num_kv_heads % 4 == 0 && 4 * G <= 16) return 4;
  return num_kv_heads % 2 == 0 && 2 * G <= 16 ? 2 : 1;
}

// Workgroups per sequence of the base / fixed-split walk (grid.y): one per kv
// head group at D = 64 (heads_per_workgroup), else one per kv head and 16-head
// slice of its query heads.
inline int walk_grid_y(int num_heads, int num_kv_heads, int head_dim) {
  const int G = num_heads / num_kv_heads;
  const int heads = head_dim == 64 ? heads_per_workgroup(num_kv_heads, G) : 1;
  return heads > 1 ? num_kv_heads / heads : num_kv_heads * ((G + 15) / 16);
}

}  // namespace pd
