// Host-side driver for the sanitizer test: the staging entry points' host
// copies (ec::copy_rect, ec::gather_rows, ec::scatter_units in
// megatron-lm_amd/csrc/host_copy.cpp)
// over odd pitches, widths, row counts and thread counts, against a plain
// loop, under AddressSanitizer and UndefinedBehaviorSanitizer.  Buffers are
// allocated to the exact extent each call may touch, so a read or write past
// a row's end is caught.  Exit 0 = all checks hold.
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <vector>

#include "host_copy.h"

#define FAIL(...) do { fprintf(stderr, __VA_ARGS__); fputc('\n', stderr); return 1; } while (0)

static uint8_t pattern(uint64_t r, uint64_t x) { return (uint8_t)(r * 131u + x * 7u + 1u); }

int main() {
  const uint32_t rows_list[] = {1, 2, 3, 7, 16};
  const uint64_t width_list[] = {1, 3, 15, 16, 17, 255, 4099};
  const uint64_t pad_list[] = {0, 1, 13, 64};
  const int thread_list[] = {1, 2, 3, 5, 8, 17, 64};
  int cases = 0;
  for (uint32_t rows : rows_list)
    for (uint64_t width : width_list)
      for (uint64_t spad : pad_list)
        for (int threads : thread_list) {
          const uint64_t dpad = (spad * 3 + 5) % 17;
          const uint64_t sp = width + spad, dp = width + dpad;
          // exactly the bytes of rows - 1 full pitches plus one row
          std::vector<uint8_t> src((rows - 1) * sp + width), dst((rows - 1) * dp + width, 0xEE);
          for (uint32_t r = 0; r < rows; ++r)
            for (uint64_t x = 0; x < width; ++x) src[r * sp + x] = pattern(r, x);
          ec::copy_rect(dst.data(), dp, src.data(), sp, rows, width, threads);
          for (uint32_t r = 0; r < rows; ++r) {
            for (uint64_t x = 0; x < width; ++x)
              if (dst[r * dp + x] != pattern(r, x))
                FAIL("copy_rect rows %u width %lu pad %lu threads %d: byte (%u, %lu)", rows,
                     (unsigned long)width, (unsigned long)spad, threads, r, (unsigned long)x);
            if (r + 1 < rows)
              for (uint64_t x = width; x < dp; ++x)
                if (dst[r * dp + x] != 0xEE) FAIL("copy_rect wrote a pitch gap");
          }
          // gather: columns [x0, x0 + width) of separately allocated rows
          const uint64_t x0 = spad;
          std::vector<std::vector<uint8_t>> rowbufs(rows);
          std::vector<const uint8_t*> ptrs(rows);
          for (uint32_t r = 0; r < rows; ++r) {
            rowbufs[r].resize(x0 + width);
            for (uint64_t x = 0; x < x0 + width; ++x) rowbufs[r][x] = pattern(r + 9, x);
            ptrs[r] = rowbufs[r].data();
          }
          std::vector<uint8_t> packed(rows * width);
          ec::gather_rows(packed.data(), ptrs.data(), x0, rows, width, threads);
          for (uint32_t r = 0; r < rows; ++r)
            for (uint64_t x = 0; x < width; ++x)
              if (packed[r * width + x] != pattern(r + 9, x0 + x)) FAIL("gather_rows byte");
          ++cases;
        }
  // scatter: a stripe-major (stripes, positions, unit) block, walked in
  // chunks of every size class (within a unit, across units and stripes),
  // into separately allocated position rows of exactly stripes * unit bytes
  const uint32_t pos_list[] = {1, 3, 16};
  const uint32_t stripe_list[] = {1, 2, 5};
  const uint64_t unit_list[] = {1, 7, 64, 4099};
  for (uint32_t positions : pos_list)
    for (uint32_t stripes : stripe_list)
      for (uint64_t unit : unit_list) {
        const uint64_t total = (uint64_t)stripes * positions * unit;
        std::vector<uint8_t> block(total);
        for (uint64_t g = 0; g < total; ++g) block[g] = pattern(g / unit, g % unit);
        const uint64_t chunk_list[] = {1, 13, unit, unit * positions + 5, total};
        for (uint64_t chunk : chunk_list)
          for (int threads : {1, 3, 8, 64}) {
            if ((total + chunk - 1) / chunk > 300) continue;  // bounded thread start-ups
            std::vector<std::vector<uint8_t>> rowbufs(positions);
            std::vector<uint8_t*> ptrs(positions);
            for (uint32_t p = 0; p < positions; ++p) {
              rowbufs[p].assign(stripes * unit, 0xEE);
              ptrs[p] = rowbufs[p].data();
            }
            for (uint64_t x0 = 0; x0 < total; x0 += chunk) {
              const uint64_t len = chunk < total - x0 ? chunk : total - x0;
              // the chunk as its own exact-size buffer, as a pinned half holds it
              std::vector<uint8_t> piece(block.begin() + x0, block.begin() + x0 + len);
              ec::scatter_units(ptrs.data(), positions, unit, x0, piece.data(), len, threads);
            }
            for (uint32_t p = 0; p < positions; ++p)
              for (uint32_t st = 0; st < stripes; ++st)
                for (uint64_t x = 0; x < unit; ++x)
                  if (rowbufs[p][st * unit + x] != pattern((uint64_t)st * positions + p, x))
                    FAIL("scatter_units positions %u stripes %u unit %lu chunk %lu threads %d: "
                         "row %u stripe %u byte %lu", positions, stripes, (unsigned long)unit,
                         (unsigned long)chunk, threads, p, st, (unsigned long)x);
            ++cases;
          }
      }
  // zero rows or width: no access at all
  ec::copy_rect(nullptr, 0, nullptr, 0, 0, 16, 4);
  ec::gather_rows(nullptr, nullptr, 0, 3, 0, 4);
  ec::scatter_units(nullptr, 3, 16, 0, nullptr, 0, 4);
  printf("sanitize copy driver ok: %d cases\n", cases);
  return 0;
}
