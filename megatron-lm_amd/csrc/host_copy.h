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

// Bytes [x0, x0 + len) of a stripe-major block of units (unit u = stripe
// u / positions, position u % positions, `unit` bytes each), held at src,
// go to their place in the position rows: byte g of the block lands at
// dst_rows[(g / unit) % positions] + (g / unit / positions) * unit + g % unit.
// Split into equal byte shares over `threads` host threads.
void scatter_units(uint8_t* const* dst_rows, uint32_t positions, uint64_t unit, uint64_t x0,
                   const uint8_t* src, uint64_t len, int threads);

}  // namespace ec
