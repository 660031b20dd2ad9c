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

}  // namespace pd
