// staging.cpp — host side of moving coded checkpoint slices out of HBM
// (ec_stage_to_host) and back in (ec_stage_to_device); the host copies are
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

#include "ec_mi355.h"
#include "host_copy.h"

extern "C" {

int ec_stage_to_host(const uint8_t* d_src, uint64_t src_pitch, uint8_t* h_dst,
                     uint64_t dst_pitch, uint32_t rows, uint64_t row_bytes, uint8_t* h_pinned,
                     uint64_t pinned_bytes, int threads, ec_stream_t stream) {
  if (rows == 0 || row_bytes == 0) return EC_OK;
  if (!d_src || !h_dst || !h_pinned || threads < 1 || threads > 64) return EC_EINVAL;
  if (src_pitch < row_bytes || dst_pitch < row_bytes) return EC_EINVAL;
  // Two halves of the pinned buffer, each holding `width` bytes of every row.
  const uint64_t half = pinned_bytes / 2;
  uint64_t width = half / rows;
  if (width >= 4096) width -= width % 4096;  // whole pages when there is room
  if (width == 0) return EC_EINVAL;
  width = std::min(width, row_bytes);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  // The events belong on the stream's device, whichever device the calling
  // thread has current.
  int prev = 0;
  hipDevice_t sdev = 0;
  if (hipGetDevice(&prev) != hipSuccess) return EC_EHIP;
  if (st && hipStreamGetDevice(st, &sdev) != hipSuccess) return EC_EHIP;
  const bool switched = st && sdev != prev;
  if (switched && hipSetDevice(sdev) != hipSuccess) return EC_EHIP;
  hipEvent_t ev[2] = {nullptr, nullptr};
  int status = EC_OK;
  for (auto& e : ev)
    if (hipEventCreateWithFlags(&e, hipEventDisableTiming | hipEventBlockingSync) != hipSuccess)
      status = EC_EHIP;
  const uint64_t n_chunks = (row_bytes + width - 1) / width;
  // Chunk j: columns [j * width, min(row_bytes, (j + 1) * width)) of every
  // row, through pinned half j % 2.  The transfer of chunk j is in flight
  // while the threads copy chunk j - 1 out of the other half.
  for (uint64_t j = 0; status == EC_OK && j <= n_chunks; ++j) {
    if (j < n_chunks) {
      const uint64_t x0 = j * width, w = std::min(width, row_bytes - x0);
      uint8_t* pin = h_pinned + (j % 2) * half;
      for (uint32_t r = 0; r < rows && status == EC_OK; ++r)
        if (hipMemcpyAsync(pin + (uint64_t)r * w, d_src + (uint64_t)r * src_pitch + x0, w,
                           hipMemcpyDeviceToHost, st) != hipSuccess)
          status = EC_EHIP;
      if (status == EC_OK && hipEventRecord(ev[j % 2], st) != hipSuccess) status = EC_EHIP;
    }
    if (status == EC_OK && j >= 1) {
      const uint64_t p = j - 1, x0 = p * width, w = std::min(width, row_bytes - x0);
      if (hipEventSynchronize(ev[p % 2]) != hipSuccess) {
        status = EC_EHIP;
        break;
      }
      ec::copy_rect(h_dst + x0, dst_pitch, h_pinned + (p % 2) * half, w, rows, w, threads);
    }
  }
  if (status != EC_OK) (void)hipStreamSynchronize(st);  // no transfer outlives the call
  for (auto& e : ev)
    if (e) (void)hipEventDestroy(e);
  if (switched) (void)hipSetDevice(prev);
  return status;
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
  uint64_t width = half / rows;
  if (width >= 4096) width -= width % 4096;
  if (width == 0) return EC_EINVAL;
  width = std::min(width, row_bytes);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  int prev = 0;
  hipDevice_t sdev = 0;
  if (hipGetDevice(&prev) != hipSuccess) return EC_EHIP;
  if (st && hipStreamGetDevice(st, &sdev) != hipSuccess) return EC_EHIP;
  const bool switched = st && sdev != prev;
  if (switched && hipSetDevice(sdev) != hipSuccess) return EC_EHIP;
  hipEvent_t ev[2] = {nullptr, nullptr};
  int status = EC_OK;
  for (auto& e : ev)
    if (hipEventCreateWithFlags(&e, hipEventDisableTiming | hipEventBlockingSync) != hipSuccess)
      status = EC_EHIP;
  const uint64_t n_chunks = (row_bytes + width - 1) / width;
  // Chunk j: the threads fill pinned half j % 2 (once the transfer of chunk
  // j - 2 out of it has landed), then the transfer is enqueued; the fill of
  // chunk j + 1 overlaps it.
  for (uint64_t j = 0; status == EC_OK && j < n_chunks; ++j) {
    const uint64_t x0 = j * width, w = std::min(width, row_bytes - x0);
    uint8_t* pin = h_pinned + (j % 2) * half;
    if (j >= 2 && hipEventSynchronize(ev[j % 2]) != hipSuccess) {
      status = EC_EHIP;
      break;
    }
    // rows x w bytes, split over the threads by equal shares of bytes
    ec::gather_rows(pin, h_rows, x0, rows, w, threads);
    for (uint32_t r = 0; r < rows && status == EC_OK; ++r)
      if (hipMemcpyAsync(d_dst + (uint64_t)r * dst_pitch + x0, pin + (uint64_t)r * w, w,
                         hipMemcpyHostToDevice, st) != hipSuccess)
        status = EC_EHIP;
    if (status == EC_OK && hipEventRecord(ev[j % 2], st) != hipSuccess) status = EC_EHIP;
  }
  // no transfer outlives the call: the pinned buffer is the caller's again
  if (hipStreamSynchronize(st) != hipSuccess && status == EC_OK) status = EC_EHIP;
  for (auto& e : ev)
    if (e) (void)hipEventDestroy(e);
  if (switched) (void)hipSetDevice(prev);
  return status;
}

}  // extern "C"
