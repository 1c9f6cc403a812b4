// ec_update.hip — ec_parity_update (update_kernel of ec_update.h for
// k <= 16, m <= 4) and the batched kernels for wide codes
// (batched_wide_kernel, update_wide_kernel: k at run time, up to
// EC_MAX_K x EC_MAX_M), which ec_batched.hip and ec_batched_copy.hip reach
// through batched_wide().
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <array>
#include <utility>

#include "ec_device.h"
#include "ec_update.h"

namespace ec {
namespace {

// --------------------------------------- batched kernels for wide codes --
// The batched encode/decode and the parity update for codes past the
// instantiated fast path (k > 16 or m > 4): k at run time, M a template
// parameter, one 16-byte chunk per lane (4 KiB tiles).  A workgroup stages
// its stripe's descriptors and the m x k tables in LDS; fast tiles issue the
// unit loads in groups of kWideGroup, edge tiles take the units one at a
// time with byte-granular ends, as in the fixed-size kernels.

struct BatchWideArgs {
  const uint64_t* dptr;  // [n_stripes][k] (update: new units, 0 = unchanged)
  const uint32_t* dlen;  // [n_stripes][k]
  const uint64_t* optr;  // update: [n_stripes][k] old units; otherwise unused
  const uint64_t* pptr;  // [n_stripes][m]
  const uint32_t* olen;  // [n_stripes][m] valid output bytes, or null = whole units
  uint8_t coeff[EC_MAX_M * EC_MAX_K];  // row-major m x k
  uint32_t unit_bytes;
  uint32_t tiles_per_unit;
  uint32_t tiles_per_block;
  uint32_t blocks_per_unit;
  FastDiv by_blocks;  // division by blocks_per_unit
  int k;
};

template <int M>
struct WideStripe {
  PermTab tab[M * EC_MAX_K];
  const uint8_t* d[EC_MAX_K];
  const uint8_t* o[EC_MAX_K];
  uint32_t len[EC_MAX_K];
  uint8_t* p[M];
  uint32_t plen[M];
};

// Tables and stripe s's descriptors into LDS.  Returns, after a barrier,
// whether any unit or output address is not 16-byte aligned (uniform).
// Lanes 0..k-1 read the data descriptors, lanes 32..32+M-1 the parity ones
// (k <= 32, M <= 16): B >= 64.
template <int M, int B>
__device__ __forceinline__ bool stage_wide(WideStripe<M>& w, const BatchWideArgs& a, uint32_t s,
                                           bool update) {
  static_assert(B >= 64, "stage_wide needs lanes 0..47");
  const int k = a.k;
  const uint32_t t = threadIdx.x;
  for (uint32_t i = t; i < (uint32_t)(M * k); i += B) w.tab[i] = dev_perm_tab(a.coeff[i]);
  if (t < (uint32_t)k) {
    // Dense arrays: the length (and in an update the old unit's address) is
    // read together with the address, not after it.
    const uint8_t* d = reinterpret_cast<const uint8_t*>(a.dptr[(uint64_t)s * k + t]);
    const uint32_t dl = a.dlen[(uint64_t)s * k + t];
    const uint8_t* o0 = update ? reinterpret_cast<const uint8_t*>(a.optr[(uint64_t)s * k + t])
                               : nullptr;
    const uint32_t l = d ? dl : 0u;
    const uint8_t* o = d ? o0 : nullptr;
    w.d[t] = d;
    w.o[t] = o;
    w.len[t] = l < a.unit_bytes ? l : a.unit_bytes;
  } else if (t >= 32 && t < 32 + M) {
    const uint32_t i = t - 32;
    uint8_t* p = reinterpret_cast<uint8_t*>(a.pptr[(uint64_t)s * M + i]);
    const uint32_t l = p ? (a.olen ? a.olen[(uint64_t)s * M + i] : a.unit_bytes) : 0u;
    w.p[i] = p;
    w.plen[i] = l < a.unit_bytes ? l : a.unit_bytes;
  }
  __syncthreads();
  uintptr_t bits = 0;
  for (int j = 0; j < k; ++j)
    bits |= reinterpret_cast<uintptr_t>(w.d[j]) | reinterpret_cast<uintptr_t>(w.o[j]);
#pragma unroll
  for (int i = 0; i < M; ++i) bits |= reinterpret_cast<uintptr_t>(w.p[i]);
  return (bits & 15u) != 0;
}

template <int M>
__device__ __forceinline__ void wide_mac(uint32_t (&acc)[M][4], const uint4& x,
                                         const PermTab* col, int k) {
  Fields f[4];
#pragma unroll
  for (int dd = 0; dd < 4; ++dd) f[dd] = fields(word(x, dd));
#pragma unroll
  for (int i = 0; i < M; ++i) {
    asm volatile("" ::: "memory");
    const PermTab t = col[i * k];
#pragma unroll
    for (int dd = 0; dd < 4; ++dd) acc[i][dd] = mac1(acc[i][dd], t, f[dd]);
  }
}

template <int M, int B>
__global__ void __launch_bounds__(B) batched_wide_kernel(const BatchWideArgs a) {
  constexpr uint32_t kWideTile = B * 16u;
  __shared__ WideStripe<M> w;
  const uint32_t s = fast_div(blockIdx.x, a.by_blocks);
  const uint32_t t0 = (blockIdx.x - s * a.blocks_per_unit) * a.tiles_per_block;
  const uint32_t t1 = min(t0 + a.tiles_per_block, a.tiles_per_unit);
  const bool misaligned = stage_wide<M, B>(w, a, s, false);
  const int k = a.k;
  for (uint32_t t = t0; t < t1; ++t) {
    const uint32_t lo = t * kWideTile, hi = lo + kWideTile;
    const uint32_t off = lo + threadIdx.x * 16u;
    bool edge = misaligned;
    for (int j = 0; j < k; ++j) edge |= w.len[j] > lo && w.len[j] < hi;
#pragma unroll
    for (int i = 0; i < M; ++i) edge |= w.plen[i] < hi;
    uint32_t acc[M][4] = {};
    if (!edge) {
      for (int j0 = 0; j0 < k; j0 += kWideGroup) {
        uint4 x[kWideGroup];
#pragma unroll
        for (int g = 0; g < kWideGroup; ++g) {
          const int j = j0 + g;
          x[g] = j < k && w.len[j] >= hi ? load_stream(w.d[j] + off) : make_uint4(0, 0, 0, 0);
        }
#pragma unroll
        for (int g = 0; g < kWideGroup; ++g) {
          if (j0 + g >= k) break;
          wide_mac<M>(acc, x[g], &w.tab[j0 + g], k);
        }
      }
#pragma unroll
      for (int i = 0; i < M; ++i)
        store_stream(w.p[i] + off, make_uint4(acc[i][0], acc[i][1], acc[i][2], acc[i][3]));
    } else {
      if (off >= a.unit_bytes) continue;
#pragma unroll 1
      for (int j = 0; j < k; ++j) {
        if (off >= w.len[j]) continue;
        wide_mac<M>(acc, load_unit(w.d[j], off, w.len[j]), &w.tab[j], k);
      }
#pragma unroll
      for (int i = 0; i < M; ++i)
        if (off < w.plen[i])
          store_unit_len(w.p[i], off, w.plen[i],
                         make_uint4(acc[i][0], acc[i][1], acc[i][2], acc[i][3]));
    }
  }
}

// parity[s][i] ^= C[i][j] * (new[s][j] ^ old[s][j]) for the changed units.
template <int M, int B>
__global__ void __launch_bounds__(B) update_wide_kernel(const BatchWideArgs a) {
  constexpr uint32_t kWideTile = B * 16u;
  __shared__ WideStripe<M> w;
  const uint32_t s = fast_div(blockIdx.x, a.by_blocks);
  const uint32_t t0 = (blockIdx.x - s * a.blocks_per_unit) * a.tiles_per_block;
  const uint32_t t1 = min(t0 + a.tiles_per_block, a.tiles_per_unit);
  stage_wide<M, B>(w, a, s, true);
  const int k = a.k;
  uint32_t longest = 0;   // past the longest changed unit the delta is zero
  for (int j = 0; j < k; ++j) longest = w.len[j] > longest ? w.len[j] : longest;
  for (uint32_t t = t0; t < t1; ++t) {
    const uint32_t off = t * kWideTile + threadIdx.x * 16u;
    if (off >= longest) continue;
    uint32_t acc[M][4] = {};
    uint4 pv[M];  // the parity does not depend on the delta: load it first
#pragma unroll
    for (int i = 0; i < M; ++i) pv[i] = load_unit(w.p[i], off, a.unit_bytes);
#pragma unroll 1
    for (int j = 0; j < k; ++j) {
      if (w.d[j] == nullptr || off >= w.len[j]) continue;  // unchanged unit, or past its end
      const uint4 vn = load_unit(w.d[j], off, w.len[j]);
      const uint4 vo = load_unit(w.o[j], off, w.len[j]);
      wide_mac<M>(acc, make_uint4(vn.x ^ vo.x, vn.y ^ vo.y, vn.z ^ vo.z, vn.w ^ vo.w),
                  &w.tab[j], k);
    }
#pragma unroll
    for (int i = 0; i < M; ++i)
      store_unit(w.p[i], off, make_uint4(pv[i].x ^ acc[i][0], pv[i].y ^ acc[i][1],
                                         pv[i].z ^ acc[i][2], pv[i].w ^ acc[i][3]));
  }
}

// The update's launch shape (update_kernel in ec_update.h): lanes per
// workgroup, 16-byte chunks per lane, and log2 of the interleaved slices of
// the grid (0: launch order).  Measured on MI355X for config 5's 1 % update
// (RS(12,4), 3,152 changed 64 KiB units in 2,993 stripes, 1.98 GB of
// traffic), microseconds per launch by lanes x chunks and slices 1 / 8:
//   256 x 1  322.8 / 311.3     256 x 2  331.6 / 322.0     256 x 4  328.4 / 324.5
//   128 x 1  331.5 / 309.7     128 x 2  331.0 / 319.6
//    64 x 1  311.3 / 308.6      64 x 2  365.4 / 320.2      64 x 4  334.1 / 324.5
// and 64 x 1 over 4 / 16 / 32 slices 307.2 / 314.0 / 315.8: one wavefront on
// a 1 KiB tile in 4 slices, 0.806 of the HBM roofline against 0.767 for the
// former 256 x 1 in launch order.  More chunks per lane (more loads in
// flight per lane, fewer workgroups) lost everywhere.
constexpr int kUpdateBlock = 64;
constexpr int kUpdateChunks = 1;
constexpr uint32_t kUpdateSliceShift = 2;

template <int K, int M>
int update_fast(const uint8_t* coeff, const uint64_t* nptr, const uint64_t* optr,
                const uint32_t* len, const uint64_t* pptr, uint32_t n_stripes,
                uint32_t unit_bytes, hipStream_t st) {
  return launch_update<K, M, kUpdateBlock, kUpdateChunks>(coeff, nptr, optr, len, pptr, n_stripes,
                                                          unit_bytes, kUpdateSliceShift, st);
}

// Wide codes through the batched kernels: encode / decode (update = false,
// optr unused) or the parity update, with B-lane workgroups on B * 16-byte
// tiles: the encode walks spans of `span` bytes (0: span_bytes()) keeping at
// least 2048 workgroups, the update one tile per workgroup.
template <int M, int B>
int launch_batched_wide_b(const uint8_t* coeff, int k, const uint64_t* dptr, const uint32_t* dlen,
                          const uint64_t* optr, const uint64_t* pptr, const uint32_t* olen,
                          uint32_t n_stripes, uint32_t unit_bytes, bool update, hipStream_t st,
                          uint32_t span) {
  BatchWideArgs a;
  a.dptr = dptr;
  a.dlen = dlen;
  a.optr = optr;
  a.pptr = pptr;
  a.olen = olen;
  for (int t = 0; t < M * k; ++t) a.coeff[t] = coeff[t];
  a.k = k;
  a.unit_bytes = unit_bytes;
  a.tiles_per_unit = (unit_bytes / 16u + B - 1) / B;
  const uint64_t total_tiles = (uint64_t)n_stripes * a.tiles_per_unit;
  uint64_t tpb = 1;
  if (!update) {
    tpb = (span ? span : span_bytes(unit_bytes)) / (B * 16u);
    if (tpb < 1) tpb = 1;
    if (total_tiles / tpb < 2048) tpb = total_tiles / 2048;
  } else {
    tpb = (total_tiles + 0x3fffffffull) >> 30;
  }
  if (tpb < 1) tpb = 1;
  if (tpb > a.tiles_per_unit) tpb = a.tiles_per_unit;
  a.tiles_per_block = (uint32_t)tpb;
  a.blocks_per_unit = (a.tiles_per_unit + a.tiles_per_block - 1) / a.tiles_per_block;
  a.by_blocks = make_fastdiv(a.blocks_per_unit);
  const uint64_t blocks = (uint64_t)n_stripes * a.blocks_per_unit;
  if (blocks > 0x7fffffffull) return EC_ERANGE;
  if (update)
    hipLaunchKernelGGL((update_wide_kernel<M, B>), dim3((unsigned)blocks), dim3(B), 0, st, a);
  else
    hipLaunchKernelGGL((batched_wide_kernel<M, B>), dim3((unsigned)blocks), dim3(B), 0, st, a);
  return hip_status();
}

// Encode and decode with m <= 4 run one-wavefront workgroups on one 1 KiB
// tile each, like the fixed-size batched kernel; wider outputs and the update
// keep 256-lane workgroups.  Both keep launch order for every unit size:
// the fixed-size kernel's 8 slices for large units (SpanGrid) gained nothing
// here and cost RS(16,6) over 4 MiB units 11 % (encode 0.606 -> 0.539 of the
// roofline; RS(20,4) 4 MiB 0.661 -> 0.659, RS(24,8) 2 MiB 0.498 -> 0.496;
// the 1 % update of RS(12,4) and RS(8,2) over 4 MiB units within 1 %).  Measured on MI355X (HBM traffic, GB/s, 8 GiB
// buffers): RS(20,4) over 4 MiB units encode 5041 -> 5314, decode of 4
// positions 4886 -> 5136; with m >= 6 the per-workgroup table build (m * k
// tables) made one-wavefront workgroups 5 % slower (RS(16,6) over 64 KiB
// units 4995 -> 4747, RS(24,8) over 1 MiB units 3980 -> 3815).
template <int M>
int launch_batched_wide(const uint8_t* coeff, int k, const uint64_t* dptr, const uint32_t* dlen,
                        const uint64_t* optr, const uint64_t* pptr, const uint32_t* olen,
                        uint32_t n_stripes, uint32_t unit_bytes, bool update, hipStream_t st) {
  if (M <= 4 && !update)
    return launch_batched_wide_b<M, 64>(coeff, k, dptr, dlen, optr, pptr, olen, n_stripes,
                                        unit_bytes, update, st, 64 * 16);
  return launch_batched_wide_b<M, kBlock>(coeff, k, dptr, dlen, optr, pptr, olen, n_stripes,
                                          unit_bytes, update, st, 0);
}

using UpdFn = int (*)(const uint8_t*, const uint64_t*, const uint64_t*, const uint32_t*,
                      const uint64_t*, uint32_t, uint32_t, hipStream_t);

template <int K, int... Ms>
constexpr auto upd_row(std::integer_sequence<int, Ms...>) {
  return std::array<UpdFn, sizeof...(Ms)>{&update_fast<K, Ms + 1>...};
}
template <int... Ks>
constexpr auto upd_table(std::integer_sequence<int, Ks...>) {
  return std::array<std::array<UpdFn, kFastMaxM>, sizeof...(Ks)>{
      upd_row<Ks + 1>(std::make_integer_sequence<int, kFastMaxM>{})...};
}
const auto kUpdTable = upd_table(std::make_integer_sequence<int, kFastMaxK>{});
using BatchWideFn = int (*)(const uint8_t*, int, const uint64_t*, const uint32_t*,
                            const uint64_t*, const uint64_t*, const uint32_t*, uint32_t, uint32_t,
                            bool, hipStream_t);
template <int... Ms>
constexpr auto batch_wide_table(std::integer_sequence<int, Ms...>) {
  return std::array<BatchWideFn, sizeof...(Ms)>{&launch_batched_wide<Ms + 1>...};
}
const auto kBatchWideTable = batch_wide_table(std::make_integer_sequence<int, EC_MAX_M>{});


}  // namespace

int batched_wide(int m, const uint8_t* coeff, int k, const uint64_t* dptr, const uint32_t* dlen,
                 const uint64_t* optr, const uint64_t* pptr, const uint32_t* olen,
                 uint32_t n_stripes, uint32_t unit_bytes, bool update, hipStream_t st) {
  if (m < 1 || m > EC_MAX_M || k < 1 || k > EC_MAX_K) return EC_ERANGE;
  return kBatchWideTable[m - 1](coeff, k, dptr, dlen, optr, pptr, olen, n_stripes, unit_bytes,
                                update, st);
}

}  // namespace ec

extern "C" {

int ec_parity_update(const uint8_t* coeff, int k, int m, const uint64_t* d_new_ptrs,
                     const uint64_t* d_old_ptrs, const uint32_t* d_len,
                     const uint64_t* d_parity_ptrs, uint32_t n_stripes, uint32_t unit_bytes,
                     ec_stream_t stream) {
  int s = ec::check_batch(coeff, k, m, d_new_ptrs, d_old_ptrs, d_parity_ptrs, unit_bytes);
  if (s != EC_OK) return s;
  if (!d_len) return EC_EINVAL;
  if (n_stripes == 0) return EC_OK;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (!ec::fast_shape(k, m))
    return ec::kBatchWideTable[m - 1](coeff, k, d_new_ptrs, d_len, d_old_ptrs, d_parity_ptrs,
                                      nullptr, n_stripes, unit_bytes, true, st);
  return ec::kUpdTable[k - 1][m - 1](coeff, d_new_ptrs, d_old_ptrs, d_len, d_parity_ptrs,
                                     n_stripes, unit_bytes, st);
}

}  // extern "C"
