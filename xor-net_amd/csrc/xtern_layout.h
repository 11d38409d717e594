// Host-side repack into the device tile layout.
#pragma once
#include <stddef.h>
#include <stdint.h>

#include <string>
#include <vector>

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
// XorSparse compact stream (XT_XORSPARSE_STREAM): the row blob re-laid for
// the device by 16-row group G and 64-column block b --
//   seg   [ng][nb]      u32: bit offset of (G, b)'s sign segment
//   mask  [ng][nb][16]  u64: the rows' block masks (rows past N: 0)
//   sign  u32 words: for each (G, b), the 16 rows' set-order sign bits one
//         after the other (row j's popcount(mask) bits, first set lane
//         first; bit 1 = negative), no padding between segments
// so the bytes read are the blob's masks and signs (the blob's per-block
// byte padding and row headers dropped) plus 4 bytes per 1024 weights.
struct XsLayout {
    int64_t nb = 0, ng = 0;
    size_t seg_off = 0, mask_off = 0, sign_off = 0, sign_bytes = 0, total = 0;
};
// Validates the blob as repack() does for XT_XORSPARSE.  Returns 0, or -1
// with *err set.
int build_xs_stream(int64_t K, int64_t N, const uint8_t* blob, size_t nbytes,
                    std::vector<uint8_t>* out, XsLayout* lay, std::string* err);
// Int8Linear::new (bits 8: out [N][K] i8) / Int4Linear::new (bits 4: out
// [N][ceil(K/2)] nibbles) with per-row scales.
int int_quantize(int bits, const float* w, int64_t N, int64_t K, uint8_t* out, float* scales);
}  // namespace xt
