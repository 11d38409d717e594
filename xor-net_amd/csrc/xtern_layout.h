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
// HF prepacked (output-dim striped) bytes [N/f][K] -> input-dim packed rows
// [N][ceil(K/f)], f = 4 (fmt 0) or 5 (fmt 1).  Returns 0, or -1 with *err set.
int hf_destripe(int fmt, int64_t K, int64_t N, const uint8_t* stored, size_t nbytes,
                uint8_t* out, std::string* err);
// Int8Linear::new (bits 8: out [N][K] i8) / Int4Linear::new (bits 4: out
// [N][ceil(K/2)] nibbles) with per-row scales.
int int_quantize(int bits, const float* w, int64_t N, int64_t K, uint8_t* out, float* scales);
}  // namespace xt
