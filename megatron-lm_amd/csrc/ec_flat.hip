// ec_flat.hip — the flat-shard kernels and entry points of the C ABI:
// ec_xor_encode, ec_rs_encode, ec_rs_decode (k equal-size shards in, m out),
// and ec_stream_create / ec_stream_destroy.  Helpers, the GF multiply and
// the streaming accesses are in ec_device.h.
#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <array>
#include <utility>
#include <vector>

#include "ec_device.h"

namespace ec {
namespace {

// ------------------------------------------------ fast matrix-vector kernel --
// parity_i = XOR_j C[i][j] * data_j over n16 16-byte chunks; all pointers
// 16-byte aligned.  Encode and decode both run this kernel (decode with the
// host-inverted rows over the survivors).

template <int K, int M>
struct RsArgs {
  const uint8_t* data[K];
  uint8_t* out[M];
  PermTab tab[M][K];
  uint64_t n16;
};

// Lanes per workgroup of the flat kernels: one wavefront for the small codes
// (tables in registers, k * m <= 20), two for the wider ones, with
// workgroups in launch order: workgroup b streams 1 or 2 KiB of every shard
// at column b * BLOCK, and the round-robin dispatch over the 8 XCDs deals
// consecutive 1-2 KiB columns to different XCDs.  Measured on MI355X over
// 256 MiB shards (HBM traffic, GB/s; the former 256-lane workgroups that
// streamed each shard at two places half a shard apart first): RS(6,3) 5887 -> 6404 (one wave),
// 6309 (two waves); RS(8,2) 5900 -> 6319 / 6381; RS(4,1) 5942 -> 6347 /
// 6377; RS(12,4) 5687 -> 6087 / 6253; RS(16,4) over 128 MiB 6116 -> 6291 /
// 6335.  RS(6,3) with one wave over 64 MiB to 1 GiB shards: 6393-6547
// (5657-6097 before).  Smaller workgroups also made the rate less dependent
// on the box: the 256-lane kernel ran RS(6,3) at 393 to 424 us per launch on
// three boxes, the 64/128-lane ones at 376 to 386.  The two-window order lost
// with them (RS(6,3) one wave: 6202 vs 6404 at 256 MiB), and so did
// interleaved slices, workgroup b taking column (b mod 2^s) * ceil(n / 2^s) +
// b / 2^s (RS(6,3) over 6 x 256 MiB, us per launch, one box: launch order
// 373, 8 slices, one per XCD, 378-381, 32 slices 406, 256 slices 447).
template <int K, int M>
constexpr int flat_block() {
  return K * M <= 20 ? 64 : 128;
}

// Three forms of the same kernel, chosen per code by flat_form:
//  - kFormLanes: a per-lane grid-stride loop over 16-byte chunks, global nt
//    loads and stores (each lane computes its own 64-bit addresses);
//  - kFormPass: workgroup b codes the B chunks at chunk b * B of every shard
//    in one pass, global nt loads and stores on a wave-uniform base (kernel
//    argument plus b * B * 16, a scalar) plus the lane's 16-byte offset;
//  - kFormPassSc1: the same with nt+sc1 buffer stores on that base
//    (store_wave).
// The pass forms cover shards up to 16 GiB in one grid (grid_of); PASSES
// adds a wave-uniform grid-stride loop for larger ones (the loop costs
// 0.5-1 % where it is not needed: RS(6,3) over 6 x 256 MiB 372.9 us
// loop-free against 376.3 with the loop).
enum FlatForm : int { kFormLanes = 0, kFormPass = 1, kFormPassSc1 = 2 };

// Every shape with k <= 16, m <= 4 was timed in all three forms over 128 MiB
// shards on two boxes (HIP events, 3 interleaved rounds each).  A pass form
// is used where it beat kFormLanes by at least 0.5 % on the mean of both
// boxes (time relative to kFormLanes):
//   kFormPassSc1: RS(1,1) 0.981, RS(1,2) 0.972, RS(1,3) 0.988, RS(4,3) 0.991,
//                 RS(4,4) 0.984, RS(5,3) 0.993, RS(6,3) 0.992
//   kFormPass:    RS(1,4) 0.982, RS(4,1) 0.988, RS(7,2) 0.982, RS(12,1) 0.993,
//                 RS(13,1) 0.989, RS(16,1) 0.960
// kFormLanes was ahead for most codes with k >= 7 (by up to 3-4 %: RS(10,3)
// 1.022 / 1.041 for the pass forms, RS(9,2) 1.025 / 1.029), and the rest lie
// within 0.5 %.  The headline shape, RS(6,3) over 6 x 256 MiB, on one box:
// 375.9 us in the former library (kFormLanes) against 371.2 in this one
// (kFormPassSc1).
template <int K, int M>
constexpr int flat_form() {
  constexpr int kSc1[][2] = {{1, 1}, {1, 2}, {1, 3}, {4, 3}, {4, 4}, {5, 3}, {6, 3}};
  constexpr int kPass[][2] = {{1, 4}, {4, 1}, {7, 2}, {12, 1}, {13, 1}, {16, 1}};
  for (const auto& p : kSc1)
    if (p[0] == K && p[1] == M) return kFormPassSc1;
  for (const auto& p : kPass)
    if (p[0] == K && p[1] == M) return kFormPass;
  return kFormLanes;
}

template <int K, int M, int FORM, bool PASSES>
__global__ void __launch_bounds__((flat_block<K, M>())) rs_kernel(const RsArgs<K, M> a) {
  constexpr int B = flat_block<K, M>();
  __shared__ PermTab tab[M][K];
  {
    // M * K <= 64 tables: one per lane of the first B lanes, looped for
    // B = 64 < M * K
    for (int q = threadIdx.x; q < M * K; q += B) tab[q / K][q % K] = a.tab[q / K][q % K];
    __syncthreads();
  }
  if constexpr (FORM == kFormLanes) {
    const uint64_t stride = (uint64_t)gridDim.x * B;
    for (uint64_t idx = (uint64_t)blockIdx.x * B + threadIdx.x; idx < a.n16; idx += stride) {
      uint4 x[K];
#pragma unroll
      for (int j = 0; j < K; ++j) x[j] = load_stream(a.data[j] + idx * 16);
      uint32_t acc[M][4] = {};
      gf_matvec16<K, M>(acc, x, tab);
#pragma unroll
      for (int i = 0; i < M; ++i)
        store_stream(a.out[i] + idx * 16, make_uint4(acc[i][0], acc[i][1], acc[i][2], acc[i][3]));
    }
  } else {
    const uint64_t stride = PASSES ? (uint64_t)gridDim.x * B : 0;
    for (uint64_t base = (uint64_t)blockIdx.x * B; base < a.n16; base += stride) {
      if (base + threadIdx.x < a.n16) {
        const uint32_t lane = threadIdx.x * 16u;
        uint4 x[K];
#pragma unroll
        for (int j = 0; j < K; ++j) x[j] = load_stream(a.data[j] + base * 16 + lane);
        uint32_t acc[M][4] = {};
        gf_matvec16<K, M>(acc, x, tab);
#pragma unroll
        for (int i = 0; i < M; ++i) {
          const uint4 v = make_uint4(acc[i][0], acc[i][1], acc[i][2], acc[i][3]);
          if constexpr (FORM == kFormPassSc1)
            store_wave<kPolicyNt | kPolicySc1>(a.out[i] + base * 16, lane, v);
          else
            store_stream(a.out[i] + base * 16 + lane, v);
        }
      }
      if (!PASSES) break;
    }
  }
}

// ------------------------------------------------------------- XOR kernel --

template <int K>
struct XorArgs {
  const uint8_t* data[K];
  uint8_t* out;
  uint64_t n16;
};

__device__ __forceinline__ uint4 xor3v(const uint4& a, const uint4& b, const uint4& c) {
  return make_uint4(xor3(a.x, b.x, c.x), xor3(a.y, b.y, c.y), xor3(a.z, b.z, c.z),
                    xor3(a.w, b.w, c.w));
}

// XOR parity: one-wavefront workgroups in launch order, one chunk per lane,
// nt buffer loads on the workgroup's wave-uniform base (as the pass forms of
// rs_kernel address it).  Measured on MI355X for XOR(4) (HBM traffic, GB/s):
// over 64 MiB shards 6482 vs 6357 for the former 512-lane workgroups with two
// chunks per lane (6399 with 128 lanes, 6288 with 256); over 256 MiB 6621 vs
// 6555.  The parity store of k > 1 is an sc1 buffer store.  XOR(4) over
// 4 x 64 MiB, same box: global nt loads with a plain global store 52.7 us,
// with an sc1 buffer store 50.9, nt buffer loads with the sc1 buffer store
// 48.9; on another box nt+sc1 stores took 54.8 us against 50.5 for sc1 ones
// (a plain store had beaten a streaming one: 6470 against 6360 GB/s).  The
// copy (k = 1) keeps the streaming global store, whose measured alternatives
// were within 1 %.
constexpr int kXorBlock = 64;

template <int K, bool PASSES>
__global__ void __launch_bounds__(kXorBlock) xor_kernel(const XorArgs<K> a) {
  const uint64_t stride = PASSES ? (uint64_t)gridDim.x * kXorBlock : 0;
  for (uint64_t base = (uint64_t)blockIdx.x * kXorBlock; base < a.n16; base += stride) {
    if (base + threadIdx.x < a.n16) {
      const uint32_t lane = threadIdx.x * 16u;
      uint4 x[K];
#pragma unroll
      for (int j = 0; j < K; ++j) x[j] = load_wave(a.data[j] + base * 16, lane);
      uint4 acc = x[0];
      int j = 1;
#pragma unroll
      for (; j + 1 < K; j += 2) acc = xor3v(acc, x[j], x[j + 1]);
      if (j < K)
        acc = make_uint4(acc.x ^ x[j].x, acc.y ^ x[j].y, acc.z ^ x[j].z, acc.w ^ x[j].w);
      if (K == 1)
        store_stream(a.out + base * 16 + lane, acc);
      else
        store_wave<kPolicySc1>(a.out + base * 16, lane, acc);
    }
    if (!PASSES) break;
  }
}

// --------------------------------------------------------- generic kernel --
// Any k <= EC_MAX_K, m <= EC_MAX_M and any alignment: byte loads and stores,
// four bytes per lane, permute tables built in LDS by the workgroup.  Used for
// shard counts beyond the instantiated ones, misaligned pointers and the
// sub-16-byte tail of the fast kernels.

struct GenArgs {
  const uint8_t* data[EC_MAX_K];
  uint8_t* out[EC_MAX_M];
  uint8_t coeff[EC_MAX_M * EC_MAX_K];
  uint64_t n;
  int k, m;
};

__global__ void __launch_bounds__(kBlock) generic_kernel(const GenArgs a) {
  __shared__ PermTab tab[EC_MAX_M * EC_MAX_K];
  for (int t = threadIdx.x; t < a.m * a.k; t += kBlock) tab[t] = dev_perm_tab(a.coeff[t]);
  __syncthreads();
  const uint64_t n4 = (a.n + 3) / 4;
  const uint64_t stride = (uint64_t)gridDim.x * kBlock;
  for (uint64_t q = (uint64_t)blockIdx.x * kBlock + threadIdx.x; q < n4; q += stride) {
    const uint64_t b0 = q * 4;
    const int nb = (int)((a.n - b0) < 4 ? (a.n - b0) : 4);
    uint32_t acc[EC_MAX_M];
    for (int i = 0; i < a.m; ++i) acc[i] = 0;
    for (int j = 0; j < a.k; ++j) {
      uint32_t w = 0;
      for (int b = 0; b < nb; ++b) w |= (uint32_t)a.data[j][b0 + b] << (8 * b);
      const Fields f = fields(w);
      for (int i = 0; i < a.m; ++i) acc[i] = mac1(acc[i], tab[i * a.k + j], f);
    }
    for (int i = 0; i < a.m; ++i)
      for (int b = 0; b < nb; ++b) a.out[i][b0 + b] = (uint8_t)(acc[i] >> (8 * b));
  }
}

// ------------------------------------------------------------ wide kernel --
// Codes past the instantiated fast path: see kWideGroup in ec_device.h.
struct WideArgs {
  const uint8_t* data[EC_MAX_K];
  uint8_t* out[EC_MAX_M];
  uint8_t coeff[EC_MAX_M * EC_MAX_K];  // row-major m x k
  uint64_t n16;
  int k;
};

// 128-lane workgroups in launch order.  Measured on MI355X (HBM traffic,
// GB/s; the former 256-lane workgroups that streamed each shard at two
// places half a shard apart first): RS(20,4) over 256 MiB 5157 -> 5464, RS(24,4) 5124 ->
// 5385, RS(10,6) over 128 MiB 5280 -> 5311, RS(6,8) 4844 -> 4902, RS(32,16)
// over 64 MiB 2720 -> 2700 (VALU-bound there).
constexpr int kWideBlock = 128;

template <int M>
__global__ void __launch_bounds__(kWideBlock) wide_kernel(const WideArgs a) {
  __shared__ PermTab tab[M * EC_MAX_K];
  const int k = a.k;
  for (int t = threadIdx.x; t < M * k; t += kWideBlock) tab[t] = dev_perm_tab(a.coeff[t]);
  __syncthreads();
  const uint64_t stride = (uint64_t)gridDim.x * kWideBlock;
  for (uint64_t idx = (uint64_t)blockIdx.x * kWideBlock + threadIdx.x;
       idx < a.n16; idx += stride) {
    uint32_t acc[M][4] = {};
    for (int j0 = 0; j0 < k; j0 += kWideGroup) {
      uint4 x[kWideGroup];
#pragma unroll
      for (int g = 0; g < kWideGroup; ++g)
        x[g] = j0 + g < k ? load_realign(a.data[j0 + g], idx * 16) : make_uint4(0, 0, 0, 0);
#pragma unroll
      for (int g = 0; g < kWideGroup; g += kWidePair<M>()) {
        if (j0 + g >= k) break;
        if constexpr (kWidePair<M>() == 2) {
          // Two coefficients per step (three XOR3 instead of two XOR3 and
          // two XOR).  x[g + 1] is zero past k and a zero byte's products
          // are zero, so the pair form is exact for an odd k as well.
          Fields fa[4], fb[4];
#pragma unroll
          for (int dd = 0; dd < 4; ++dd) {
            fa[dd] = fields(word(x[g], dd));
            fb[dd] = fields(word(x[g + 1], dd));
          }
          const int jb = j0 + g + 1 < k ? j0 + g + 1 : j0 + g;
#pragma unroll
          for (int i = 0; i < M; ++i) {
            // Read each table right before its uses (see gf_matvec16).
            asm volatile("" ::: "memory");
            const PermTab ta = tab[i * k + j0 + g], tb = tab[i * k + jb];
#pragma unroll
            for (int dd = 0; dd < 4; ++dd) acc[i][dd] = mac2(acc[i][dd], ta, fa[dd], tb, fb[dd]);
          }
        } else {
          Fields f[4];
#pragma unroll
          for (int dd = 0; dd < 4; ++dd) f[dd] = fields(word(x[g], dd));
#pragma unroll
          for (int i = 0; i < M; ++i) {
            asm volatile("" ::: "memory");
            const PermTab t = tab[i * k + j0 + g];
#pragma unroll
            for (int dd = 0; dd < 4; ++dd) acc[i][dd] = mac1(acc[i][dd], t, f[dd]);
          }
        }
      }
    }
#pragma unroll
    for (int i = 0; i < M; ++i)
      store_stream(a.out[i] + idx * 16, make_uint4(acc[i][0], acc[i][1], acc[i][2], acc[i][3]));
  }
}

// ---------------------------------------------------------- host launch --

template <int K, int M>
int launch_rs(const uint8_t* coeff, const uint8_t* const* d, uint8_t* const* o, uint64_t n16,
              hipStream_t st) {
  RsArgs<K, M> a;
  for (int j = 0; j < K; ++j) a.data[j] = d[j];
  for (int i = 0; i < M; ++i) a.out[i] = o[i];
  for (int i = 0; i < M; ++i)
    for (int j = 0; j < K; ++j) a.tab[i][j] = perm_tab(coeff[i * K + j]);
  a.n16 = n16;
  constexpr int B = flat_block<K, M>();
  constexpr int F = flat_form<K, M>();
  const unsigned grid = grid_of(n16, B);
  if constexpr (F == kFormLanes) {
    hipLaunchKernelGGL((rs_kernel<K, M, F, false>), dim3(grid), dim3(B), 0, st, a);
  } else {
    if ((uint64_t)grid * B >= n16)
      hipLaunchKernelGGL((rs_kernel<K, M, F, false>), dim3(grid), dim3(B), 0, st, a);
    else
      hipLaunchKernelGGL((rs_kernel<K, M, F, true>), dim3(grid), dim3(B), 0, st, a);
  }
  return hip_status();
}

template <int M>
int launch_wide(const uint8_t* coeff, int k, const uint8_t* const* d, uint8_t* const* o,
                uint64_t n16, hipStream_t st) {
  WideArgs a;
  for (int j = 0; j < k; ++j) a.data[j] = d[j];
  for (int i = 0; i < M; ++i) a.out[i] = o[i];
  for (int t = 0; t < M * k; ++t) a.coeff[t] = coeff[t];
  a.n16 = n16;
  a.k = k;
  hipLaunchKernelGGL((wide_kernel<M>), dim3(grid_of(n16, kWideBlock)), dim3(kWideBlock), 0, st, a);
  return hip_status();
}

template <int K>
int launch_xor(const uint8_t* const* d, uint8_t* o, uint64_t n16, hipStream_t st) {
  XorArgs<K> a;
  for (int j = 0; j < K; ++j) a.data[j] = d[j];
  a.out = o;
  a.n16 = n16;
  const unsigned grid = grid_of(n16, kXorBlock);
  if ((uint64_t)grid * kXorBlock >= n16)
    hipLaunchKernelGGL((xor_kernel<K, false>), dim3(grid), dim3(kXorBlock), 0, st, a);
  else
    hipLaunchKernelGGL((xor_kernel<K, true>), dim3(grid), dim3(kXorBlock), 0, st, a);
  return hip_status();
}

using RsFn = int (*)(const uint8_t*, const uint8_t* const*, uint8_t* const*, uint64_t,
                     hipStream_t);
using XorFn = int (*)(const uint8_t* const*, uint8_t*, uint64_t, hipStream_t);

template <int K, int... Ms>
constexpr auto rs_row(std::integer_sequence<int, Ms...>) {
  return std::array<RsFn, sizeof...(Ms)>{&launch_rs<K, Ms + 1>...};
}
template <int... Ks>
constexpr auto rs_table(std::integer_sequence<int, Ks...>) {
  return std::array<std::array<RsFn, kFastMaxM>, sizeof...(Ks)>{
      rs_row<Ks + 1>(std::make_integer_sequence<int, kFastMaxM>{})...};
}
template <int... Ks>
constexpr auto xor_table(std::integer_sequence<int, Ks...>) {
  return std::array<XorFn, sizeof...(Ks)>{&launch_xor<Ks + 1>...};
}
using WideFn = int (*)(const uint8_t*, int, const uint8_t* const*, uint8_t* const*, uint64_t,
                       hipStream_t);
template <int... Ms>
constexpr auto wide_table(std::integer_sequence<int, Ms...>) {
  return std::array<WideFn, sizeof...(Ms)>{&launch_wide<Ms + 1>...};
}

const auto kRsTable = rs_table(std::make_integer_sequence<int, kFastMaxK>{});
const auto kXorTable = xor_table(std::make_integer_sequence<int, kFastMaxK>{});
const auto kWideTable = wide_table(std::make_integer_sequence<int, EC_MAX_M>{});

int launch_generic(const uint8_t* coeff, int k, int m, const uint8_t* const* d,
                   uint8_t* const* o, uint64_t offset, uint64_t n, hipStream_t st) {
  GenArgs a;
  for (int j = 0; j < k; ++j) a.data[j] = d[j] + offset;
  for (int i = 0; i < m; ++i) a.out[i] = o[i] + offset;
  for (int t = 0; t < m * k; ++t) a.coeff[t] = coeff[t];
  a.n = n;
  a.k = k;
  a.m = m;
  const uint64_t n4 = (n + 3) / 4;
  uint64_t blocks = (n4 + kBlock - 1) / kBlock;
  if (blocks > 4096) blocks = 4096;
  hipLaunchKernelGGL(generic_kernel, dim3((unsigned)(blocks ? blocks : 1)), dim3(kBlock), 0, st,
                     a);
  return hip_status();
}

// Common misalignment of a set of addresses modulo 16, or -1 if they differ.
inline int common_skew(const uint8_t* const* a, int n, int skew) {
  for (int i = 0; i < n; ++i) {
    const int s = (int)(reinterpret_cast<uintptr_t>(a[i]) & 15u);
    if (skew < 0) skew = s;
    else if (s != skew) return -1;
  }
  return skew;
}

int matvec(const uint8_t* coeff, int k, int m, const uint8_t* const* d, uint8_t* const* o,
           uint64_t nbytes, hipStream_t st) {
  if (!coeff || !d || !o) return EC_EINVAL;
  if (k < 1 || m < 1) return EC_EINVAL;
  if (k > EC_MAX_K || m > EC_MAX_M) return EC_ERANGE;
  if (nbytes == 0) return EC_OK;  // empty shards may have null addresses
  for (int j = 0; j < k; ++j)
    if (!d[j]) return EC_EINVAL;
  for (int i = 0; i < m; ++i)
    if (!o[i]) return EC_EINVAL;
  // The outputs fix the frame: the bytes up to their next 16-byte boundary
  // run through the byte kernel, the 16-byte columns after it through a
  // vector kernel (the fast one when every input shares the outputs'
  // misalignment, else the wide one, which realigns each input), and the
  // last partial column through the byte kernel.  Outputs of different
  // misalignments take the byte kernel throughout.
  const int skew = common_skew(o, m, -1);
  if (skew < 0) return launch_generic(coeff, k, m, d, o, 0, nbytes, st);
  const bool same = common_skew(d, k, skew) == skew;
  uint64_t head = skew ? 16u - (uint64_t)skew : 0;
  if (head > nbytes) head = nbytes;
  int s = EC_OK;
  if (head) s = launch_generic(coeff, k, m, d, o, 0, head, st);
  const uint64_t n16 = (nbytes - head) / 16;
  if (s == EC_OK && n16) {
    const uint8_t* da[EC_MAX_K];
    uint8_t* oa[EC_MAX_M];
    for (int j = 0; j < k; ++j) da[j] = d[j] + head;
    for (int i = 0; i < m; ++i) oa[i] = o[i] + head;
    if (same && k <= kFastMaxK && m <= kFastMaxM)
      s = kRsTable[k - 1][m - 1](coeff, da, oa, n16, st);
    else
      s = kWideTable[m - 1](coeff, k, da, oa, n16, st);
  }
  const uint64_t done = head + n16 * 16;
  if (s == EC_OK && done < nbytes) s = launch_generic(coeff, k, m, d, o, done, nbytes - done, st);
  return s;
}

}  // namespace
}  // namespace ec

extern "C" {

int ec_xor_encode(const uint8_t* const* d_data, int k, uint8_t* d_parity, uint64_t nbytes,
                  ec_stream_t stream) {
  if (!d_data || k < 1) return EC_EINVAL;
  if (k > EC_MAX_K) return EC_ERANGE;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (nbytes == 0) return EC_OK;  // empty shards may have null addresses
  if (!d_parity) return EC_EINVAL;
  for (int j = 0; j < k; ++j)
    if (!d_data[j]) return EC_EINVAL;
  uint8_t ones[EC_MAX_K];
  for (int j = 0; j < k; ++j) ones[j] = 1;  // 1*x = x: XOR parity via the generic path
  uint8_t* const out[1] = {d_parity};
  const int skew = ec::common_skew(out, 1, -1);
  const bool same = ec::common_skew(d_data, k, skew) == skew;
  uint64_t head = skew ? 16u - (uint64_t)skew : 0;
  if (head > nbytes) head = nbytes;
  int s = EC_OK;
  if (head) s = ec::launch_generic(ones, k, 1, d_data, out, 0, head, st);
  const uint64_t n16 = (nbytes - head) / 16;
  if (s == EC_OK && n16) {
    const uint8_t* da[EC_MAX_K];
    for (int j = 0; j < k; ++j) da[j] = d_data[j] + head;
    uint8_t* const oa[1] = {d_parity + head};
    s = same && k <= ec::kFastMaxK ? ec::kXorTable[k - 1](da, d_parity + head, n16, st)
                                   : ec::kWideTable[0](ones, k, da, oa, n16, st);
  }
  const uint64_t done = head + n16 * 16;
  if (s == EC_OK && done < nbytes)
    s = ec::launch_generic(ones, k, 1, d_data, out, done, nbytes - done, st);
  return s;
}

int ec_rs_encode(const uint8_t* coeff, int k, int m, const uint8_t* const* d_data,
                 uint8_t* const* d_parity, uint64_t nbytes, ec_stream_t stream) {
  return ec::matvec(coeff, k, m, d_data, d_parity, nbytes, reinterpret_cast<hipStream_t>(stream));
}

int ec_rs_decode(const uint8_t* rows, int k, int e, const uint8_t* const* d_survivors,
                 uint8_t* const* d_out, uint64_t nbytes, ec_stream_t stream) {
  return ec::matvec(rows, k, e, d_survivors, d_out, nbytes, reinterpret_cast<hipStream_t>(stream));
}

int ec_stream_create(int device, int n_cus, ec_stream_t* out) {
  if (!out) return EC_EINVAL;
  *out = nullptr;
  int count = 0;
  if (hipGetDeviceCount(&count) != hipSuccess) return EC_EHIP;
  if (device < 0 || device >= count) return EC_EINVAL;
  int cus = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess ||
      cus <= 0)
    return EC_EHIP;
  const int n = (n_cus <= 0 || n_cus > cus) ? cus : n_cus;
  std::vector<uint32_t> mask((cus + 31) / 32, 0u);
  for (int c = 0; c < n; ++c) mask[c / 32] |= 1u << (c % 32);
  int prev = 0;
  if (hipGetDevice(&prev) != hipSuccess) return EC_EHIP;
  if (prev != device && hipSetDevice(device) != hipSuccess) return EC_EHIP;
  hipStream_t st = nullptr;
  const hipError_t e =
      hipExtStreamCreateWithCUMask(&st, static_cast<uint32_t>(mask.size()), mask.data());
  if (prev != device) (void)hipSetDevice(prev);
  if (e != hipSuccess) {
    (void)hipGetLastError();
    return EC_EHIP;
  }
  *out = st;
  return EC_OK;
}

int ec_stream_destroy(ec_stream_t stream) {
  if (!stream) return EC_EINVAL;
  return hipStreamDestroy(reinterpret_cast<hipStream_t>(stream)) == hipSuccess ? EC_OK : EC_EHIP;
}

}  // extern "C"
