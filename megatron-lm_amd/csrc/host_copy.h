// host_copy.h — the multi-threaded host memory copies of the staging entry
// points (staging.cpp): no HIP calls, so the same code builds on its own
// with g++ for the sanitizer test.
#pragma once

#include <stdint.h>

namespace ec {

// dst[r * dst_pitch + x] = src[r * src_pitch + x] for r < rows, x < width,
// split into equal byte shares (whole rows, or column ranges of a row) over
// `threads` host threads (1 <= threads <= 64).
void copy_rect(uint8_t* dst, uint64_t dst_pitch, const uint8_t* src, uint64_t src_pitch,
               uint32_t rows, uint64_t width, int threads);

// dst[r * width + x] = src_rows[r][x0 + x] for r < rows, x < width: columns
// [x0, x0 + width) of `rows` separate host rows packed back to back, split
// into equal byte shares over `threads` host threads.
void gather_rows(uint8_t* dst, const uint8_t* const* src_rows, uint64_t x0, uint32_t rows,
                 uint64_t width, int threads);

}  // namespace ec
