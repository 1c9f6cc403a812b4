// staging.cpp — host side of moving coded checkpoint slices out of HBM
// (ec_stage_to_host for row-major regions, ec_stage_stripes_to_host for a
// stripe-major block) and back in (ec_stage_to_device); the host copies are
// in host_copy.cpp.
//
// A background save stages the coded block to host memory while training
// runs in the same process.  The whole loop (a transfer per chunk, a wait,
// host copies on several threads) runs inside one foreign call, which
// ctypes makes with the interpreter's lock released, so the staging thread
// takes that lock from the training thread only to start and to finish.
//
// The two device-to-host calls move their bytes with one of the GPU's SDMA
// copy engines (the ROCr copy API, forced onto an engine), not with HIP
// transfers, when both buffers are runtime allocations.  HIP runs device-to-host transfers as copy kernels on the
// stream's hardware queue, and it spreads streams over a few queues: when
// the staging stream's queue was training's, its 1 GiB copies ran in order
// between training's kernels, and a save cost a training loop 6-91 ms
// instead of 6-13 ms with the engine; the link rate is the same.  (On a
// CU-masked stream the HIP transfers also held the host; a copy kernel
// writing the pinned buffer through its device address, on a stream of its
// own, slowed training's steps by up to 2.3x, also on a few CUs.)  The
// upload of the load path (ec_stage_to_device), which holds its caller
// anyway, keeps HIP transfers on the caller's stream.
#include <hip/hip_runtime.h>
#include <hsa/hsa.h>
#include <hsa/hsa_ext_amd.h>
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

// ---- Copies on an SDMA engine (ec_stage_stripes_to_host) ----

enum class Owner { kNone, kFits, kShort };

// Where [p, p + bytes) lies: kFits when inside one allocation ROCr made
// (hipMalloc, hipHostMalloc and torch's allocators over them) whose owner
// is a `type` agent, stored in *agent; kShort when p is in such an
// allocation that ends before p + bytes; kNone otherwise (memory ROCr did
// not allocate, such as pageable or virtually mapped memory).
Owner owner_of(const void* p, uint64_t bytes, hsa_device_type_t type, hsa_agent_t* agent) {
  hsa_amd_pointer_info_t pi = {};
  pi.size = sizeof(pi);
  if (hsa_amd_pointer_info(p, &pi, nullptr, nullptr, nullptr) != HSA_STATUS_SUCCESS ||
      pi.type != HSA_EXT_POINTER_TYPE_HSA)
    return Owner::kNone;
  hsa_device_type_t t;
  if (hsa_agent_get_info(pi.agentOwner, HSA_AGENT_INFO_DEVICE, &t) != HSA_STATUS_SUCCESS ||
      t != type)
    return Owner::kNone;
  const uint8_t* base = static_cast<const uint8_t*>(
      type == HSA_DEVICE_TYPE_CPU && pi.hostBaseAddress ? pi.hostBaseAddress
                                                        : pi.agentBaseAddress);
  const uint8_t* q = static_cast<const uint8_t*>(p);
  if (!base || q < base || (uint64_t)(q - base) >= pi.sizeInBytes) return Owner::kNone;
  if (bytes > pi.sizeInBytes - (uint64_t)(q - base)) return Owner::kShort;
  *agent = pi.agentOwner;
  return Owner::kFits;
}

// Two completion signals (one per pinned half) and the engine chosen for
// device-to-host copies; the signals are destroyed, after every copy has
// landed, when it goes out of scope.  ROCr, the runtime under HIP, is open
// once HIP is (the Session's HIP calls come first); the library takes no
// reference of its own on it, so its teardown at exit stays HIP's.  Were it
// not open, the pointer queries fail and the call takes HIP transfers.
struct EngineCopies {
  hsa_agent_t gpu = {0}, cpu = {0};
  hsa_amd_sdma_engine_id_t engine = HSA_AMD_SDMA_ENGINE_0;
  hsa_signal_t sig[2] = {{0}, {0}};
  bool busy[2] = {false, false};
  bool ready = false;

  // EC_OK with ready set when the block and the pinned buffer both lie in
  // ROCr allocations (device, then host) and an engine can copy between
  // them; EC_OK with ready clear when not (the caller uses HIP transfers);
  // EC_EINVAL when d_block's allocation ends before the block does.
  int setup(const uint8_t* d_block, uint64_t block_bytes, uint8_t* h_pinned,
            uint64_t pinned_bytes) {
    const Owner dev = owner_of(d_block, block_bytes, HSA_DEVICE_TYPE_GPU, &gpu);
    if (dev == Owner::kShort) return EC_EINVAL;
    if (dev != Owner::kFits ||
        owner_of(h_pinned, pinned_bytes, HSA_DEVICE_TYPE_CPU, &cpu) != Owner::kFits)
      return EC_OK;
    uint32_t mask = 0;
    if (hsa_amd_memory_copy_engine_status(cpu, gpu, &mask) != HSA_STATUS_SUCCESS || mask == 0)
      return EC_OK;
    engine = static_cast<hsa_amd_sdma_engine_id_t>(mask & (0u - mask));  // the lowest one
    for (auto& s : sig)
      if (hsa_signal_create(0, 0, nullptr, &s) != HSA_STATUS_SUCCESS) return EC_OK;
    ready = true;
    return EC_OK;
  }
  // Arms signal h for the n copies that fill pinned half h.
  void arm(int h, uint32_t n) {
    hsa_signal_store_relaxed(sig[h], n);
    busy[h] = true;
  }
  // Starts the copy of w bytes from src into dst; it completes on signal h
  // (armed).  False if the runtime refused it: then forgo() the copies of
  // the half that were never started.
  bool copy(int h, uint8_t* dst, const uint8_t* src, uint64_t w) {
    return hsa_amd_memory_async_copy_on_engine(dst, cpu, src, gpu, w, 0, nullptr, sig[h], engine,
                                               true) == HSA_STATUS_SUCCESS;
  }
  void forgo(int h, uint32_t n) { hsa_signal_subtract_relaxed(sig[h], n); }
  // Blocks (asleep) until signal h's copy has landed.
  void wait(int h) {
    if (!busy[h]) return;
    while (hsa_signal_wait_scacquire(sig[h], HSA_SIGNAL_CONDITION_LT, 1, UINT64_MAX,
                                     HSA_WAIT_STATE_BLOCKED) >= 1) {
    }
    busy[h] = false;
  }
  ~EngineCopies() {
    for (int h = 0; h < 2; ++h) wait(h);
    for (auto& s : sig)
      if (s.handle) hsa_signal_destroy(s);
  }
};

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
  // The device region: rows - 1 pitches and one row.
  if (rows > 1 && src_pitch > (UINT64_MAX - row_bytes) / (rows - 1)) return EC_EINVAL;
  const uint64_t src_span = (uint64_t)(rows - 1) * src_pitch + row_bytes;
  Session ss(stream);
  if (!ss.ok()) return ss.status;
  EngineCopies eng;
  const int st = eng.setup(d_src, src_span, h_pinned, 2 * half);
  if (st != EC_OK) return st;
  const uint64_t n_chunks = (row_bytes + width - 1) / width;
  // Chunk j: columns [j * width, min(row_bytes, (j + 1) * width)) of every
  // row, through pinned half j % 2.  The transfer of chunk j is in flight
  // while the threads copy chunk j - 1 out of the other half.  On a copy
  // engine (as ec_stage_stripes_to_host) when both buffers allow it, else
  // HIP transfers on the stream.
  if (eng.ready) {
    if (hipStreamSynchronize(ss.st) != hipSuccess) return EC_EHIP;
    ss.stats.copy_engine = 1;
    const Clock::time_point t_dev = Clock::now();
    for (uint64_t j = 0; ss.ok() && j <= n_chunks; ++j) {
      if (j < n_chunks) {
        const uint64_t x0 = j * width, w = std::min(width, row_bytes - x0);
        const int h = (int)(j % 2);
        uint8_t* pin = h_pinned + h * half;
        eng.arm(h, rows);
        for (uint32_t r = 0; r < rows; ++r)
          if (!eng.copy(h, pin + (uint64_t)r * w, d_src + (uint64_t)r * src_pitch + x0, w)) {
            eng.forgo(h, rows - r);
            ss.fail();
            break;
          }
        ++ss.stats.chunks;
      }
      if (j >= 1 && ss.ok()) {
        const uint64_t p = j - 1, x0 = p * width, w = std::min(width, row_bytes - x0);
        const Clock::time_point t0 = Clock::now();
        eng.wait((int)(p % 2));
        const double wt = seconds_since(t0);
        ss.stats.wait_s += wt;
        ss.stats.max_wait_s = std::max(ss.stats.max_wait_s, wt);
        if (p + 1 == n_chunks) ss.stats.device_s = seconds_since(t_dev);
        ss.host_copy([&] {
          ec::copy_rect(h_dst + x0, dst_pitch, h_pinned + (p % 2) * half, w, rows, w, threads);
        });
      }
    }
    return ss.status;   // eng's destructor waits for copies still in flight
  }
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
  if (!ss.ok()) return ss.status;
  EngineCopies eng;
  const int st = eng.setup(d_block, total, h_pinned, 2 * half);
  if (st != EC_OK) return st;
  const uint64_t n_chunks = (total + width - 1) / width;
  // Chunk j: bytes [j * width, ...) of the block, contiguous on the device,
  // in one transfer to pinned half j % 2; the threads scatter chunk j - 1's
  // units into their rows meanwhile.
  if (eng.ready) {
    // The engine does not follow the stream: wait for the stream's work
    // (the coding of the block) here, then time the copies on the host.
    if (hipStreamSynchronize(ss.st) != hipSuccess) return EC_EHIP;
    ss.stats.copy_engine = 1;
    const Clock::time_point t_dev = Clock::now();
    for (uint64_t j = 0; ss.ok() && j <= n_chunks; ++j) {
      if (j < n_chunks) {
        const uint64_t x0 = j * width, w = std::min(width, total - x0);
        const int h = (int)(j % 2);
        eng.arm(h, 1);
        if (!eng.copy(h, h_pinned + h * half, d_block + x0, w)) {
          eng.forgo(h, 1);
          ss.fail();
        }
        ++ss.stats.chunks;
      }
      if (j >= 1 && ss.ok()) {
        const uint64_t p = j - 1, x0 = p * width, w = std::min(width, total - x0);
        const Clock::time_point t0 = Clock::now();
        eng.wait((int)(p % 2));
        const double wt = seconds_since(t0);
        ss.stats.wait_s += wt;
        ss.stats.max_wait_s = std::max(ss.stats.max_wait_s, wt);
        if (p + 1 == n_chunks) ss.stats.device_s = seconds_since(t_dev);
        ss.host_copy([&] {
          ec::scatter_units(h_rows, positions, unit_bytes, x0, h_pinned + (p % 2) * half, w,
                            threads);
        });
      }
    }
    return ss.status;   // eng's destructor waits for a copy still in flight
  }
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
