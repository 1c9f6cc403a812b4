// host_copy.cpp — multi-threaded host copies for the staging entry points.
#include "host_copy.h"

#include <string.h>

#include <algorithm>
#include <thread>
#include <vector>

namespace ec {
namespace {

// run(t) for t in [0, threads), share 0 on the calling thread and the others
// on threads of their own.  A thread that cannot be started (the system is
// out of threads or memory) has its share run on the calling thread, so no
// C++ exception reaches the C ABI and every started thread is joined.
template <class F>
void run_shares(int threads, const F& run) {
  std::vector<std::thread> pool;
  int t = 1;
  try {
    pool.reserve(threads - 1);
    for (; t < threads; ++t) pool.emplace_back(run, t);
  } catch (...) {
  }
  for (int u = t; u < threads; ++u) run(u);
  run(0);
  for (auto& th : pool) th.join();
}

// Share t of `total` bytes laid out as rows of `width`: calls
// piece(row, column, count) for each row fragment of bytes
// [t * share, min(total, (t + 1) * share)).
template <class P>
void for_share(int t, uint64_t total, uint64_t share, uint64_t width, const P& piece) {
  uint64_t b = (uint64_t)t * share;
  const uint64_t e = std::min(total, b + share);
  while (b < e) {
    const uint64_t r = b / width, x = b % width;
    const uint64_t n = std::min(e - b, width - x);
    piece(r, x, n);
    b += n;
  }
}

}  // namespace

void copy_rect(uint8_t* dst, uint64_t dst_pitch, const uint8_t* src, uint64_t src_pitch,
               uint32_t rows, uint64_t width, int threads) {
  if (rows == 0 || width == 0 || threads < 1) return;
  const uint64_t total = (uint64_t)rows * width;
  const uint64_t share = (total + threads - 1) / threads;
  run_shares(threads, [&](int t) {
    for_share(t, total, share, width, [&](uint64_t r, uint64_t x, uint64_t n) {
      memcpy(dst + r * dst_pitch + x, src + r * src_pitch + x, n);
    });
  });
}

void gather_rows(uint8_t* dst, const uint8_t* const* src_rows, uint64_t x0, uint32_t rows,
                 uint64_t width, int threads) {
  if (rows == 0 || width == 0 || threads < 1) return;
  const uint64_t total = (uint64_t)rows * width;
  const uint64_t share = (total + threads - 1) / threads;
  run_shares(threads, [&](int t) {
    for_share(t, total, share, width, [&](uint64_t r, uint64_t x, uint64_t n) {
      memcpy(dst + r * width + x, src_rows[r] + x0 + x, n);
    });
  });
}

void scatter_units(uint8_t* const* dst_rows, uint32_t positions, uint64_t unit, uint64_t x0,
                   const uint8_t* src, uint64_t len, int threads) {
  if (len == 0 || unit == 0 || positions == 0 || threads < 1) return;
  const uint64_t share = (len + threads - 1) / threads;
  run_shares(threads, [&](int t) {
    uint64_t b = (uint64_t)t * share;
    const uint64_t e = std::min(len, b + share);
    while (b < e) {
      const uint64_t g = x0 + b, u = g / unit, off = g % unit;
      const uint64_t n = std::min(e - b, unit - off);
      memcpy(dst_rows[u % positions] + (u / positions) * unit + off, src + b, n);
      b += n;
    }
  });
}

}  // namespace ec
