// ec_batched_copy.hip — ec_encode_batched_copy: the batched encode that also
// writes a zero-padded copy of every data unit in the same pass.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <array>
#include <utility>

#include "ec_batched.h"

namespace ec {
namespace {

// Encode plus a zero-padded copy of every data unit (cptr), same tiling.
template <int K, int M>
int launch_batched_copy(const uint8_t* coeff, const uint64_t* dptr, const uint32_t* dlen,
                        const uint64_t* pptr, const uint64_t* cptr, uint32_t n_stripes,
                        uint32_t unit_bytes, hipStream_t st) {
  return launch_batched_u<K, M, 1, true, kBatchBlock>(coeff, dptr, dlen, pptr, nullptr, cptr,
                                                      n_stripes, unit_bytes, st);
}

using BatchCopyFn = int (*)(const uint8_t*, const uint64_t*, const uint32_t*, const uint64_t*,
                            const uint64_t*, uint32_t, uint32_t, hipStream_t);
template <int K, int... Ms>
constexpr auto batch_copy_row(std::integer_sequence<int, Ms...>) {
  return std::array<BatchCopyFn, sizeof...(Ms)>{&launch_batched_copy<K, Ms + 1>...};
}
template <int... Ks>
constexpr auto batch_copy_table(std::integer_sequence<int, Ks...>) {
  return std::array<std::array<BatchCopyFn, kFastMaxM>, sizeof...(Ks)>{
      batch_copy_row<Ks + 1>(std::make_integer_sequence<int, kFastMaxM>{})...};
}
const auto kBatchCopyTable = batch_copy_table(std::make_integer_sequence<int, kFastMaxK>{});

}  // namespace
}  // namespace ec

extern "C" {

int ec_encode_batched_copy(const uint8_t* coeff, int k, int m, const uint64_t* d_data_ptrs,
                           const uint32_t* d_data_len, const uint64_t* d_parity_ptrs,
                           const uint64_t* d_copy_ptrs, uint32_t n_stripes, uint32_t unit_bytes,
                           ec_stream_t stream) {
  int s = ec::check_batch(coeff, k, m, d_data_ptrs, d_data_len, d_parity_ptrs, unit_bytes);
  if (s != EC_OK) return s;
  if (!d_copy_ptrs) return EC_EINVAL;
  if (n_stripes == 0) return EC_OK;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (ec::fast_shape(k, m))
    return ec::kBatchCopyTable[k - 1][m - 1](coeff, d_data_ptrs, d_data_len, d_parity_ptrs,
                                             d_copy_ptrs, n_stripes, unit_bytes, st);
  // Wide codes: the encode, then the copies as k * n_stripes one-unit
  // stripes of coefficient 1 (the descriptor arrays read as [n_stripes * k][1]).
  const uint64_t units = (uint64_t)n_stripes * (uint64_t)k;
  if (units > 0xffffffffull) return EC_ERANGE;
  s = ec::batched_wide(m, coeff, k, d_data_ptrs, d_data_len, nullptr, d_parity_ptrs,
                                 nullptr, n_stripes, unit_bytes, false, st);
  if (s != EC_OK) return s;
  const uint8_t one = 1;
  return ec::batched_fast(1, 1, &one, d_data_ptrs, d_data_len, d_copy_ptrs, nullptr,
                               (uint32_t)units, unit_bytes, st);
}

}  // extern "C"
