// staging.cpp — host side of moving coded checkpoint slices out of HBM
// (ec_stage_to_host for row-major regions, ec_stage_stripes_to_host for a
// stripe-major block) and back in (ec_stage_to_device); the host copies are
// in host_copy.cpp.
//
// A background save stages the coded block to host memory while training
// runs in the same process.  The whole loop (a transfer per chunk and row,
// an event wait, host copies on several threads) runs inside one foreign
// call, which ctypes makes with the interpreter's lock released, so the
// staging thread takes that lock from the training thread only to start
// and to finish.  Give it an ordinary stream: on MI355X, transfers issued
// on a CU-masked stream held the host and slowed the training kernels beside
// them; on ordinary streams they ran asynchronously without doing so.  (A
// copy kernel writing the pinned buffer through its device address, on a
// stream of its own, slowed training's steps more: by up to 2.3x, also on a
// few CUs.)
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>
#include <chrono>

#include "ec_mi355.h"
#include "host_copy.h"

namespace {

using Clock = std::chrono::steady_clock;

double seconds_since(Clock::time_point t0) {
  return std::chrono::duration<double>(Clock::now() - t0).count();
}

// The timings of this thread's last staging call (ec_stage_last_stats).
thread_local ec_stage_stats g_last_stats = {};

// The stream's device made current for the call (the events belong on it,
// whichever device the calling thread has current) and the two events that
// mark the pinned halves; undone on every return.
//
// It also keeps the call's timings: host time blocked in the waits and in
// the threads' copies, and the device time from the first transfer's start
// to the last one's end (two timing events), stored for
// ec_stage_last_stats when the call ends.
struct Session {
  hipStream_t st;
  int prev = 0;
  bool switched = false;
  hipEvent_t ev[2] = {nullptr, nullptr};
  hipEvent_t span[2] = {nullptr, nullptr};  // timing events around the transfers
  bool span_started = false, span_ended = false;
  int status = EC_OK;
  Clock::time_point start = Clock::now();
  ec_stage_stats stats = {};

  explicit Session(ec_stream_t stream) : st(reinterpret_cast<hipStream_t>(stream)) {
    hipDevice_t sdev = 0;
    if (hipGetDevice(&prev) != hipSuccess || (st && hipStreamGetDevice(st, &sdev) != hipSuccess)) {
      status = EC_EHIP;
      return;
    }
    switched = st && sdev != prev;
    if (switched && hipSetDevice(sdev) != hipSuccess) {
      switched = false;
      status = EC_EHIP;
      return;
    }
    for (auto& e : ev)
      if (hipEventCreateWithFlags(&e, hipEventDisableTiming | hipEventBlockingSync) != hipSuccess)
        status = EC_EHIP;
    for (auto& e : span)
      if (hipEventCreateWithFlags(&e, hipEventBlockingSync) != hipSuccess) status = EC_EHIP;
  }
  ~Session() {
    if (span_ended) {
      float ms = 0.0f;
      if (hipEventSynchronize(span[1]) == hipSuccess &&
          hipEventElapsedTime(&ms, span[0], span[1]) == hipSuccess)
        stats.device_s = ms * 1e-3;
    }
    stats.wall_s = seconds_since(start);
    g_last_stats = stats;
    for (auto& e : ev)
      if (e) (void)hipEventDestroy(e);
    for (auto& e : span)
      if (e) (void)hipEventDestroy(e);
    if (switched) (void)hipSetDevice(prev);
  }
  bool ok() const { return status == EC_OK; }
  void fail() { status = EC_EHIP; }
  // Before the first transfer: the start of the device-time span.
  void begin() {
    if (ok() && !span_started) {
      if (hipEventRecord(span[0], st) != hipSuccess) fail();
      span_started = true;
    }
  }
  // Marks pinned half h as filled by what is enqueued so far (one chunk).
  void mark(int h) {
    if (ok() && hipEventRecord(ev[h], st) != hipSuccess) fail();
    ++stats.chunks;
  }
  // After the last transfer: the end of the device-time span.
  void end() {
    if (ok() && span_started && hipEventRecord(span[1], st) == hipSuccess) span_ended = true;
  }
  // Waits until the transfers marked on half h have landed.
  void wait(int h) {
    const Clock::time_point t0 = Clock::now();
    if (ok() && hipEventSynchronize(ev[h]) != hipSuccess) fail();
    const double w = seconds_since(t0);
    stats.wait_s += w;
    stats.max_wait_s = std::max(stats.max_wait_s, w);
  }
  // Runs the threads' copy fn(), timed.
  template <class F>
  void host_copy(const F& fn) {
    const Clock::time_point t0 = Clock::now();
    fn();
    stats.host_copy_s += seconds_since(t0);
  }
};

// Bytes per pinned half: whole pages when there is room.
uint64_t half_of(uint64_t pinned_bytes, uint64_t per_byte_rows) {
  uint64_t w = pinned_bytes / 2 / per_byte_rows;
  if (w >= 4096) w -= w % 4096;
  return w;
}

}  // namespace

extern "C" {

int ec_stage_to_host(const uint8_t* d_src, uint64_t src_pitch, uint8_t* h_dst,
                     uint64_t dst_pitch, uint32_t rows, uint64_t row_bytes, uint8_t* h_pinned,
                     uint64_t pinned_bytes, int threads, ec_stream_t stream) {
  if (rows == 0 || row_bytes == 0) return EC_OK;
  if (!d_src || !h_dst || !h_pinned || threads < 1 || threads > 64) return EC_EINVAL;
  if (src_pitch < row_bytes || dst_pitch < row_bytes) return EC_EINVAL;
  // Two halves of the pinned buffer, each holding `width` bytes of every row.
  const uint64_t half = pinned_bytes / 2;
  uint64_t width = half_of(pinned_bytes, rows);
  if (width == 0) return EC_EINVAL;
  width = std::min(width, row_bytes);
  Session ss(stream);
  const uint64_t n_chunks = (row_bytes + width - 1) / width;
  // Chunk j: columns [j * width, min(row_bytes, (j + 1) * width)) of every
  // row, through pinned half j % 2.  The transfer of chunk j is in flight
  // while the threads copy chunk j - 1 out of the other half.
  ss.begin();
  for (uint64_t j = 0; ss.ok() && j <= n_chunks; ++j) {
    if (j < n_chunks) {
      const uint64_t x0 = j * width, w = std::min(width, row_bytes - x0);
      uint8_t* pin = h_pinned + (j % 2) * half;
      for (uint32_t r = 0; r < rows && ss.ok(); ++r)
        if (hipMemcpyAsync(pin + (uint64_t)r * w, d_src + (uint64_t)r * src_pitch + x0, w,
                           hipMemcpyDeviceToHost, ss.st) != hipSuccess)
          ss.fail();
      ss.mark(j % 2);
      if (j + 1 == n_chunks) ss.end();
    }
    if (j >= 1) {
      const uint64_t p = j - 1, x0 = p * width, w = std::min(width, row_bytes - x0);
      ss.wait(p % 2);
      if (!ss.ok()) break;
      ss.host_copy([&] {
        ec::copy_rect(h_dst + x0, dst_pitch, h_pinned + (p % 2) * half, w, rows, w, threads);
      });
    }
  }
  if (!ss.ok()) (void)hipStreamSynchronize(ss.st);  // no transfer outlives the call
  return ss.status;
}

int ec_stage_stripes_to_host(const uint8_t* d_block, uint32_t n_stripes, uint32_t positions,
                             uint64_t unit_bytes, uint8_t* const* h_rows, uint8_t* h_pinned,
                             uint64_t pinned_bytes, int threads, ec_stream_t stream) {
  if (n_stripes == 0 || positions == 0 || unit_bytes == 0) return EC_OK;
  if (!d_block || !h_rows || !h_pinned || threads < 1 || threads > 64) return EC_EINVAL;
  for (uint32_t p = 0; p < positions; ++p)
    if (!h_rows[p]) return EC_EINVAL;
  const uint64_t units = (uint64_t)n_stripes * positions;
  if (unit_bytes > UINT64_MAX / units) return EC_EINVAL;
  const uint64_t total = units * unit_bytes, half = pinned_bytes / 2;
  uint64_t width = half_of(pinned_bytes, 1);
  if (width == 0) return EC_EINVAL;
  width = std::min(width, total);
  Session ss(stream);
  const uint64_t n_chunks = (total + width - 1) / width;
  // Chunk j: bytes [j * width, ...) of the block, contiguous on the device,
  // in one transfer to pinned half j % 2; the threads scatter chunk j - 1's
  // units into their rows meanwhile.
  ss.begin();
  for (uint64_t j = 0; ss.ok() && j <= n_chunks; ++j) {
    if (j < n_chunks) {
      const uint64_t x0 = j * width, w = std::min(width, total - x0);
      if (hipMemcpyAsync(h_pinned + (j % 2) * half, d_block + x0, w, hipMemcpyDeviceToHost,
                         ss.st) != hipSuccess)
        ss.fail();
      ss.mark(j % 2);
      if (j + 1 == n_chunks) ss.end();
    }
    if (j >= 1) {
      const uint64_t p = j - 1, x0 = p * width, w = std::min(width, total - x0);
      ss.wait(p % 2);
      if (!ss.ok()) break;
      ss.host_copy([&] {
        ec::scatter_units(h_rows, positions, unit_bytes, x0, h_pinned + (p % 2) * half, w,
                          threads);
      });
    }
  }
  if (!ss.ok()) (void)hipStreamSynchronize(ss.st);  // no transfer outlives the call
  return ss.status;
}

int ec_stage_to_device(const uint8_t* const* h_rows, uint32_t rows, uint64_t row_bytes,
                       uint8_t* d_dst, uint64_t dst_pitch, uint8_t* h_pinned,
                       uint64_t pinned_bytes, int threads, ec_stream_t stream) {
  if (rows == 0 || row_bytes == 0) return EC_OK;
  if (!h_rows || !d_dst || !h_pinned || threads < 1 || threads > 64) return EC_EINVAL;
  for (uint32_t r = 0; r < rows; ++r)
    if (!h_rows[r]) return EC_EINVAL;
  if (dst_pitch < row_bytes) return EC_EINVAL;
  const uint64_t half = pinned_bytes / 2;
  uint64_t width = half_of(pinned_bytes, rows);
  if (width == 0) return EC_EINVAL;
  width = std::min(width, row_bytes);
  Session ss(stream);
  const uint64_t n_chunks = (row_bytes + width - 1) / width;
  // Chunk j: the threads fill pinned half j % 2 (once the transfer of chunk
  // j - 2 out of it has landed), then the transfer is enqueued; the fill of
  // chunk j + 1 overlaps it.
  for (uint64_t j = 0; ss.ok() && j < n_chunks; ++j) {
    const uint64_t x0 = j * width, w = std::min(width, row_bytes - x0);
    uint8_t* pin = h_pinned + (j % 2) * half;
    if (j >= 2) ss.wait(j % 2);
    if (!ss.ok()) break;
    // rows x w bytes, split over the threads by equal shares of bytes
    ss.host_copy([&] { ec::gather_rows(pin, h_rows, x0, rows, w, threads); });
    ss.begin();
    for (uint32_t r = 0; r < rows && ss.ok(); ++r)
      if (hipMemcpyAsync(d_dst + (uint64_t)r * dst_pitch + x0, pin + (uint64_t)r * w, w,
                         hipMemcpyHostToDevice, ss.st) != hipSuccess)
        ss.fail();
    ss.mark(j % 2);
    if (j + 1 == n_chunks) ss.end();
  }
  // no transfer outlives the call: the pinned buffer is the caller's again
  {
    const Clock::time_point t0 = Clock::now();
    if (hipStreamSynchronize(ss.st) != hipSuccess && ss.ok()) ss.fail();
    ss.stats.wait_s += seconds_since(t0);
  }
  return ss.status;
}

int ec_stage_last_stats(ec_stage_stats* out) {
  if (!out) return EC_EINVAL;
  *out = g_last_stats;
  return EC_OK;
}

}  // extern "C"
