// ec_batched.hip — ec_encode_batched and ec_decode_batched: one launch over
// the stripes of a ragged unit layout, k <= 16 and m <= 4 through the fully
// unrolled batched_kernel (ec_batched.h), wider codes through
// batched_wide_kernel (ec_update.hip).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <array>
#include <utility>

#include "ec_batched.h"

namespace ec {
namespace {

// One-wavefront workgroups, one 1 KiB tile each (see kBatchBlock).  The tile
// is also no larger than the smallest units that stream at HBM rate: with
// 16 KiB tiles every tile of a 4 KiB unit held the unit's end and took the
// edge path (RS(8,2) over 4 KiB units 1.7 TB/s).
template <int K, int M>
int launch_batched(const uint8_t* coeff, const uint64_t* dptr, const uint32_t* dlen,
                   const uint64_t* pptr, const uint32_t* olen, uint32_t n_stripes,
                   uint32_t unit_bytes, hipStream_t st) {
  return launch_batched_u<K, M, 1, false, kBatchBlock>(coeff, dptr, dlen, pptr, olen, nullptr,
                                                       n_stripes, unit_bytes, st);
}

using BatchFn = int (*)(const uint8_t*, const uint64_t*, const uint32_t*, const uint64_t*,
                        const uint32_t*, uint32_t, uint32_t, hipStream_t);

template <int K, int... Ms>
constexpr auto batch_row(std::integer_sequence<int, Ms...>) {
  return std::array<BatchFn, sizeof...(Ms)>{&launch_batched<K, Ms + 1>...};
}
template <int... Ks>
constexpr auto batch_table(std::integer_sequence<int, Ks...>) {
  return std::array<std::array<BatchFn, kFastMaxM>, sizeof...(Ks)>{
      batch_row<Ks + 1>(std::make_integer_sequence<int, kFastMaxM>{})...};
}
const auto kBatchTable = batch_table(std::make_integer_sequence<int, kFastMaxK>{});

}  // namespace

int batched_fast(int k, int m, const uint8_t* coeff, const uint64_t* dptr, const uint32_t* dlen,
                 const uint64_t* pptr, const uint32_t* olen, uint32_t n_stripes,
                 uint32_t unit_bytes, hipStream_t st) {
  if (!fast_shape(k, m) || k < 1 || m < 1) return EC_ERANGE;
  return kBatchTable[k - 1][m - 1](coeff, dptr, dlen, pptr, olen, n_stripes, unit_bytes, st);
}

}  // namespace ec

extern "C" {

int ec_encode_batched(const uint8_t* coeff, int k, int m, const uint64_t* d_data_ptrs,
                      const uint32_t* d_data_len, const uint64_t* d_parity_ptrs,
                      uint32_t n_stripes, uint32_t unit_bytes, ec_stream_t stream) {
  int s = ec::check_batch(coeff, k, m, d_data_ptrs, d_data_len, d_parity_ptrs, unit_bytes);
  if (s != EC_OK) return s;
  if (n_stripes == 0) return EC_OK;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (!ec::fast_shape(k, m))
    return ec::batched_wide(m, coeff, k, d_data_ptrs, d_data_len, nullptr, d_parity_ptrs,
                                      nullptr, n_stripes, unit_bytes, false, st);
  return ec::kBatchTable[k - 1][m - 1](coeff, d_data_ptrs, d_data_len, d_parity_ptrs, nullptr,
                                       n_stripes, unit_bytes, st);
}

int ec_decode_batched(const uint8_t* rows, int k, int e, const uint64_t* d_surv_ptrs,
                      const uint32_t* d_surv_len, const uint64_t* d_out_ptrs,
                      const uint32_t* d_out_len, uint32_t n_stripes, uint32_t unit_bytes,
                      ec_stream_t stream) {
  int s = ec::check_batch(rows, k, e, d_surv_ptrs, d_surv_len, d_out_ptrs, unit_bytes);
  if (s != EC_OK) return s;
  if (!d_out_len) return EC_EINVAL;
  if (n_stripes == 0) return EC_OK;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (!ec::fast_shape(k, e))
    return ec::batched_wide(e, rows, k, d_surv_ptrs, d_surv_len, nullptr, d_out_ptrs,
                                      d_out_len, n_stripes, unit_bytes, false, st);
  return ec::kBatchTable[k - 1][e - 1](rows, d_surv_ptrs, d_surv_len, d_out_ptrs, d_out_len,
                                       n_stripes, unit_bytes, st);
}

}  // extern "C"
