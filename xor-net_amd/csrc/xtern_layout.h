// Host-side repack into the device tile layout.
#pragma once
#include <stddef.h>
#include <stdint.h>

#include <string>

#include "xtern_internal.h"

namespace xt {
size_t tile_bytes(int fmt, int64_t K, int64_t N);
// Returns 0, or -1 with *err set.
int repack(int fmt, int64_t K, int64_t N, const void* src, size_t nbytes, void* dst,
           std::string* err);
}  // namespace xt
