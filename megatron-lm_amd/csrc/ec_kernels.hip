// ec_kernels.hip — gfx950 kernels and the device entry points of the C ABI:
// ec_xor_encode, ec_rs_encode, ec_rs_decode, ec_encode_batched,
// ec_decode_batched, ec_parity_update.
//
// The work is byte-wise GF(2^8) arithmetic over HBM-resident shards: it is
// bound by HBM bandwidth, not by the matrix cores, so everything here is
// VALU code laid out for streaming.
//
// Data layout and mapping.
//   A shard is a flat byte range.  Lane l of a 256-lane workgroup owns 16
//   bytes (one global_load_dwordx4) of every shard at chunk index
//   base + u*256 + l, u < U, so each wavefront reads 1 KiB contiguous per
//   shard per load and the k loads of a lane are all in flight together.
//   The m parity outputs of those bytes are accumulated in VGPRs and written
//   once: every input byte is read from HBM exactly once and every parity
//   byte written exactly once.  Loads and stores are non-temporal (streamed
//   past L2 and the Infinity Cache), and for shards below 512 MiB tiles are
//   renumbered so that the shards are streamed at two places at once
//   (tile_order).  Measured on
//   MI355X for RS(6,3) over 256 MiB shards: plain loads/stores and tables in
//   SGPRs 5.48 TB/s of HBM traffic; streaming access 5.90; plus LDS tables
//   6.15; the two-place order with one chunk per lane 6.29-6.54 over five
//   buffer layouts, where one window per XCD gave 5.69-6.22 (see
//   gf_matvec16 for the table-read order that keeps wider codes at the same
//   rate).
//
// GF multiply by a coefficient c (see PermTab in gf256.h): the byte x is cut
// into fields x[2:0], x[5:3], x[7:6]; each field indexes an 8- or 4-entry
// table of products held in one or two 32-bit registers, resolved for four
// bytes at once by one v_perm_b32.  The three partial products and the
// running parity are combined with v_bitop3_b32 (XOR3), so one coefficient
// costs 3 permutes + 1.5 XOR3 per dword, and the field selectors (5 ops per
// dword) are shared by all m outputs.
#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <array>
#include <utility>
#include <vector>

#include "ec_mi355.h"
#include "gf256.h"

namespace ec {
namespace {

constexpr int kBlock = 256;     // lanes per workgroup (4 wavefronts)
constexpr int kFastMaxK = 16;   // template-instantiated shard counts
constexpr int kFastMaxM = 4;
// Bytes of each unit a batched workgroup walks: 8 KiB for units up to
// 256 KiB, 16 KiB above, and never less than one tile.  Measured on MI355X
// (HBM traffic, two chunks per lane for k <= 8), spans of 64/32/16/8 KiB:
// RS(8,2) over 4 MiB units 5.31/5.50/5.71/5.54 TB/s; RS(8,2) over 64 KiB
// units 6.17/6.14/6.32/6.63; RS(12,4) over ragged 64 KiB units
// 5.87/5.86/6.13/6.22.  With four chunks per lane (batched_unroll, units
// that are a multiple of 16 KiB) a k <= 8 tile is 16 KiB, so those codes run
// one tile per workgroup.
inline uint32_t span_bytes(uint32_t unit_bytes) {
  return unit_bytes <= (256u << 10) ? (8u << 10) : (16u << 10);
}

// ---------------------------------------------------------------- helpers --

__device__ __forceinline__ uint32_t xor3(uint32_t a, uint32_t b, uint32_t c) {
  return __builtin_amdgcn_bitop3_b32(a, b, c, 0x96);
}

// Byte select from the 64-bit pair {hi:lo}: selector byte v in 0..7 returns
// byte v of lo (v < 4) or byte v-4 of hi.
__device__ __forceinline__ uint32_t perm(uint32_t hi, uint32_t lo, uint32_t sel) {
  return __builtin_amdgcn_perm(hi, lo, sel);
}

struct Fields {
  uint32_t f0, f1, f2;
};

__device__ __forceinline__ Fields fields(uint32_t w) {
  return {w & 0x07070707u, (w >> 3) & 0x07070707u, (w >> 6) & 0x03030303u};
}

// acc ^= c*w for the four bytes of w (single coefficient).
__device__ __forceinline__ uint32_t mac1(uint32_t acc, const PermTab& t, const Fields& f) {
  acc = xor3(acc, perm(t.hi0, t.lo0, f.f0), perm(t.hi1, t.lo1, f.f1));
  return acc ^ perm(t.t2, t.t2, f.f2);
}

// acc ^= a*wa ^ b*wb (two coefficients, six products, three XOR3).
__device__ __forceinline__ uint32_t mac2(uint32_t acc, const PermTab& a, const Fields& fa,
                                         const PermTab& b, const Fields& fb) {
  acc = xor3(acc, perm(a.hi0, a.lo0, fa.f0), perm(a.hi1, a.lo1, fa.f1));
  acc = xor3(acc, perm(a.t2, a.t2, fa.f2), perm(b.hi0, b.lo0, fb.f0));
  return xor3(acc, perm(b.hi1, b.lo1, fb.f1), perm(b.t2, b.t2, fb.f2));
}

__device__ __forceinline__ uint32_t word(const uint4& v, int d) {
  return d == 0 ? v.x : d == 1 ? v.y : d == 2 ? v.z : v.w;
}

// Streaming (non-temporal) 16-byte global accesses: every shard byte is
// touched once, so nothing is worth keeping in L2 or the Infinity Cache.
// Addresses are cast to the global address space: pointers read from
// descriptor arrays are otherwise generic and compile to flat loads.
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(1))) u32x4 global_u32x4;
typedef __attribute__((address_space(1))) uint8_t global_u8;

__device__ __forceinline__ const global_u8* gptr(const void* p) {
  return (const global_u8*)(uintptr_t)p;
}
__device__ __forceinline__ global_u8* gptr(void* p) { return (global_u8*)(uintptr_t)p; }

__device__ __forceinline__ uint4 load_stream(const void* p) {
  const u32x4 v = __builtin_nontemporal_load((const global_u32x4*)(uintptr_t)p);
  return make_uint4(v.x, v.y, v.z, v.w);
}

__device__ __forceinline__ void store_stream(void* p, const uint4& v) {
  const u32x4 w = {v.x, v.y, v.z, v.w};
  __builtin_nontemporal_store(w, (global_u32x4*)(uintptr_t)p);
}

// Two-window tile order.  Workgroups are dispatched round-robin over the 8
// XCDs (workgroup b runs on XCD b % 8).  Renumbering b -> (b % 2) * per + b / 2
// gives the even XCDs the first half of the tile range and the odd XCDs the
// second half, so every shard is streamed at two places half a shard apart.
// On MI355X, for shards below kSplitMaxBytes, this beat launch order (one
// place) and one window per XCD (eight places) for every code measured, on
// every buffer layout tried: separate allocations, one packed block, random
// 4 KiB offsets, 1 MiB and 12 KiB padding.  From 512 MiB shards on it lost
// 8-20 % to launch order (RS(6,3): 512 MiB 4.80 vs 5.65 TB/s, 1 GiB 4.93 vs
// 5.92, 2 GiB 5.06 vs 5.73; up to 448 MiB it won or tied), also with the
// halves interleaved in segments of 16-256 MiB, so larger shards keep
// launch order.  A bijection on [0, gridDim.x); an odd last tile keeps its
// index.
constexpr uint64_t kSplitMaxBytes = 512ull << 20;

__device__ __forceinline__ uint32_t split_tile(uint32_t b, uint32_t nb) {
  const uint32_t per = nb >> 1;
  return b < (per << 1) ? (b & 1u) * per + (b >> 1) : b;
}

__device__ __forceinline__ uint32_t tile_order(uint32_t b, uint32_t nb, uint64_t n16) {
  return n16 * 16 < kSplitMaxBytes ? split_tile(b, nb) : b;
}

// Copy the m x k permute tables from the kernel arguments into LDS, where
// the unrolled loops read them as wave-uniform broadcasts straight into
// VGPRs (v_perm_b32 may read only one SGPR, so tables held in SGPRs cost a
// v_mov per use and spill beyond ~100 SGPRs).
template <int K, int M>
__device__ __forceinline__ void stage_tables(PermTab (&dst)[M][K], const PermTab (&src)[M][K]) {
  const int t = threadIdx.x;
  if (t < M * K) dst[t / K][t % K] = src[t / K][t % K];
  __syncthreads();
}

// Accumulate the products of all K shards for one 16-byte chunk:
// acc[i][d] = XOR_j tab[i][j] * x[j].d
//
// Two loop orders, picked at compile time by the table footprint 5*M*K:
//  - small codes (M*K <= 20, e.g. RS(6,3), RS(8,2)): d -> j -> i, and the
//    compiler keeps every table in VGPRs for the whole kernel (<= 100
//    registers), so no LDS traffic at all in the loop;
//  - wider codes: j (in pairs) -> i -> d, the selectors of x[j], x[j+1] are
//    computed once for all outputs and each coefficient's table is read from
//    LDS once per chunk, right before its four uses.  The empty asm with a
//    memory clobber stops the compiler from hoisting those reads out of the
//    grid-stride loop: kept live in VGPRs, the tables alone would need 240
//    registers for RS(12,4) (one wave per SIMD, no latency hiding).
// Measured on MI355X (HBM traffic): RS(12,4) 3.2 TB/s with hoisted tables vs
// 5.9 with per-use reads; RS(16,4) 0.8 vs 5.3; RS(6,3) 6.0-6.2 hoisted vs
// 5.6 per-use.
template <int K, int M>
constexpr bool tables_in_registers() {
  return K * M <= 20;
}

template <int K, int M>
__device__ __forceinline__ void gf_matvec16(uint32_t (&acc)[M][4], const uint4 (&x)[K],
                                            const PermTab (&tab)[M][K]) {
  if constexpr (tables_in_registers<K, M>()) {
#pragma unroll
    for (int d = 0; d < 4; ++d) {
#pragma unroll
      for (int j = 0; j + 1 < K; j += 2) {
        const Fields fa = fields(word(x[j], d));
        const Fields fb = fields(word(x[j + 1], d));
#pragma unroll
        for (int i = 0; i < M; ++i) acc[i][d] = mac2(acc[i][d], tab[i][j], fa, tab[i][j + 1], fb);
      }
      if (K & 1) {
        const Fields f = fields(word(x[K - 1], d));
#pragma unroll
        for (int i = 0; i < M; ++i) acc[i][d] = mac1(acc[i][d], tab[i][K - 1], f);
      }
    }
  } else {
#pragma unroll
    for (int j = 0; j + 1 < K; j += 2) {
      Fields fa[4], fb[4];
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        fa[d] = fields(word(x[j], d));
        fb[d] = fields(word(x[j + 1], d));
      }
#pragma unroll
      for (int i = 0; i < M; ++i) {
        asm volatile("" ::: "memory");
        const PermTab ta = tab[i][j], tb = tab[i][j + 1];
#pragma unroll
        for (int d = 0; d < 4; ++d) acc[i][d] = mac2(acc[i][d], ta, fa[d], tb, fb[d]);
      }
    }
    if (K & 1) {
      Fields f[4];
#pragma unroll
      for (int d = 0; d < 4; ++d) f[d] = fields(word(x[K - 1], d));
#pragma unroll
      for (int i = 0; i < M; ++i) {
        asm volatile("" ::: "memory");
        const PermTab t = tab[i][K - 1];
#pragma unroll
        for (int d = 0; d < 4; ++d) acc[i][d] = mac1(acc[i][d], t, f[d]);
      }
    }
  }
}

// Device-side field multiply (shift-and-reduce), used only to build the
// permute tables of the generic kernel in LDS.
__device__ uint8_t dev_gf_mul(uint32_t a, uint32_t b) {
  uint32_t r = 0;
  for (int i = 0; i < 8; ++i) {
    if (b & 1u) r ^= a;
    b >>= 1;
    a <<= 1;
    if (a & 0x100u) a ^= 0x11Du;
  }
  return (uint8_t)r;
}

__device__ PermTab dev_perm_tab(uint32_t c) {
  PermTab p;
  uint32_t w[5] = {0, 0, 0, 0, 0};
  for (int a = 0; a < 8; ++a) {
    w[a >> 2] |= (uint32_t)dev_gf_mul(c, a) << (8 * (a & 3));
    w[2 + (a >> 2)] |= (uint32_t)dev_gf_mul(c, a << 3) << (8 * (a & 3));
  }
  for (int a = 0; a < 4; ++a) w[4] |= (uint32_t)dev_gf_mul(c, a << 6) << (8 * a);
  p.lo0 = w[0];
  p.hi0 = w[1];
  p.lo1 = w[2];
  p.hi1 = w[3];
  p.t2 = w[4];
  return p;
}

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

template <int K, int M, int U>
__global__ void __launch_bounds__(kBlock) rs_kernel(const RsArgs<K, M> a) {
  __shared__ PermTab tab[M][K];
  stage_tables<K, M>(tab, a.tab);
  const uint64_t tile = (uint64_t)kBlock * U;
  const uint64_t stride = (uint64_t)gridDim.x * tile;
  for (uint64_t base = (uint64_t)tile_order(blockIdx.x, gridDim.x, a.n16) * tile + threadIdx.x;
       base < a.n16; base += stride) {
    uint4 x[U][K];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const uint64_t idx = base + (uint64_t)u * kBlock;
      if (idx < a.n16) {
#pragma unroll
        for (int j = 0; j < K; ++j) x[u][j] = load_stream(a.data[j] + idx * 16);
      } else {
#pragma unroll
        for (int j = 0; j < K; ++j) x[u][j] = make_uint4(0, 0, 0, 0);
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const uint64_t idx = base + (uint64_t)u * kBlock;
      uint32_t acc[M][4] = {};
      gf_matvec16<K, M>(acc, x[u], tab);
      if (idx < a.n16) {
#pragma unroll
        for (int i = 0; i < M; ++i)
          store_stream(a.out[i] + idx * 16, make_uint4(acc[i][0], acc[i][1], acc[i][2], acc[i][3]));
      }
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

// XOR parity: 512-lane workgroups in launch order (measured on MI355X for
// XOR(4) over 64 MiB shards: 6.37 TB/s of HBM traffic; 6.21 with 256 lanes;
// 5.68 with one tile window per XCD and 6.00 with split_tile's two, which
// only pay off for the RS kernel).
constexpr int kXorBlock = 512;

template <int K, int U>
__global__ void __launch_bounds__(kXorBlock) xor_kernel(const XorArgs<K> a) {
  const uint64_t tile = (uint64_t)kXorBlock * U;
  const uint64_t stride = (uint64_t)gridDim.x * tile;
  for (uint64_t base = (uint64_t)blockIdx.x * tile + threadIdx.x; base < a.n16;
       base += stride) {
    uint4 x[U][K];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const uint64_t idx = base + (uint64_t)u * kXorBlock;
      if (idx < a.n16) {
#pragma unroll
        for (int j = 0; j < K; ++j) x[u][j] = load_stream(a.data[j] + idx * 16);
      } else {
#pragma unroll
        for (int j = 0; j < K; ++j) x[u][j] = make_uint4(0, 0, 0, 0);
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const uint64_t idx = base + (uint64_t)u * kXorBlock;
      uint4 acc = x[u][0];
      int j = 1;
#pragma unroll
      for (; j + 1 < K; j += 2) acc = xor3v(acc, x[u][j], x[u][j + 1]);
      if (j < K)
        acc = make_uint4(acc.x ^ x[u][j].x, acc.y ^ x[u][j].y, acc.z ^ x[u][j].z,
                         acc.w ^ x[u][j].w);
      if (idx < a.n16) {
        if (K == 1)  // a plain copy: streaming stores measured 3 % faster
          store_stream(a.out + idx * 16, acc);
        else
          reinterpret_cast<uint4*>(a.out)[idx] = acc;
      }
    }
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
// Codes past the instantiated fast path (k > 16 or m > 4, up to 32 x 16) on
// 16-byte-aligned shards: rs_kernel's column layout and tile order with the
// m outputs in registers (M is a template parameter) and k read at run time
// in groups of kWideGroup loads in flight.  The m x k tables do not fit the
// kernel arguments (10 KiB for 16 x 32), so each workgroup builds them in LDS
// from the coefficient bytes.  Measured over 256 MiB shards (HBM TB/s): a
// full grid beat grids capped at 4k-32k workgroups (RS(6,8) 5.34 vs
// 4.5-5.2, RS(24,4) 5.37 vs 4.7-4.9), so the table build costs less than the
// lost parallelism; groups of 16 loads halved the rate, groups of 4 were
// 0-15 % slower than 8.
constexpr int kWideGroup = 8;

// Coefficients per step of the wide kernel's inner loop: pairs for m >= 8,
// where the GF arithmetic bounds the kernel (RS(32,16) 2.49 -> 2.68 TB/s,
// RS(10,12) 4.03 -> 4.22), single ones below, where the pair form's longer
// dependency chains cost 2-6 % (RS(24,4) 5.13 vs 4.90).
template <int M>
constexpr int kWidePair() {
  return M >= 8 ? 2 : 1;
}

// 16 bytes at base + off, where off is a multiple of 16 and base may have any
// alignment r = base mod 16 (uniform: it depends on the shard only).  r = 0
// is one dwordx4 load; otherwise the two aligned dwordx4 that hold the bytes
// are loaded and v_alignbyte_b32 ({hi, lo} >> 8 * (byte count)) shifts them
// into place.  Both aligned
// blocks hold at least one byte of [base + off, base + off + 16), so no
// load leaves the 16-byte blocks (and pages) that the shard itself touches.
template <int Q>
__device__ __forceinline__ uint4 align_words(const uint4& lo, const uint4& hi, uint32_t sh) {
  const uint32_t w[8] = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
  return make_uint4(__builtin_amdgcn_alignbyte(w[Q + 1], w[Q], sh),
                    __builtin_amdgcn_alignbyte(w[Q + 2], w[Q + 1], sh),
                    __builtin_amdgcn_alignbyte(w[Q + 3], w[Q + 2], sh),
                    __builtin_amdgcn_alignbyte(w[Q + 4], w[Q + 3], sh));
}

__device__ __forceinline__ uint4 load_realign(const uint8_t* base, uint64_t off) {
  const uint32_t r = (uint32_t)reinterpret_cast<uintptr_t>(base) & 15u;
  if (r == 0) return load_stream(base + off);
  const uint8_t* b = base - r + off;
  const uint4 lo = load_stream(b), hi = load_stream(b + 16);
  const uint32_t sh = r & 3u;
  switch (r >> 2) {
    case 0: return align_words<0>(lo, hi, sh);
    case 1: return align_words<1>(lo, hi, sh);
    case 2: return align_words<2>(lo, hi, sh);
    default: return align_words<3>(lo, hi, sh);
  }
}

struct WideArgs {
  const uint8_t* data[EC_MAX_K];
  uint8_t* out[EC_MAX_M];
  uint8_t coeff[EC_MAX_M * EC_MAX_K];  // row-major m x k
  uint64_t n16;
  int k;
};

template <int M>
__global__ void __launch_bounds__(kBlock) wide_kernel(const WideArgs a) {
  __shared__ PermTab tab[M * EC_MAX_K];
  const int k = a.k;
  for (int t = threadIdx.x; t < M * k; t += kBlock) tab[t] = dev_perm_tab(a.coeff[t]);
  __syncthreads();
  const uint64_t stride = (uint64_t)gridDim.x * kBlock;
  for (uint64_t idx = (uint64_t)tile_order(blockIdx.x, gridDim.x, a.n16) * kBlock + threadIdx.x;
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

// ------------------------------------------------ batched stripe kernels --
// Grid = n_stripes x tiles_per_unit workgroups, stripe-major, so consecutive
// workgroups stream adjacent bytes of the same k units.  The descriptor of a
// stripe is uniform across the workgroup (scalar loads).

// 16 bytes of a unit at byte offset off, zero beyond len.  A 16-byte-aligned
// unit takes one dwordx4 load; the chunk that straddles len, and every chunk
// of a misaligned unit, is read byte by byte, so nothing past len is read.
__device__ __forceinline__ uint4 load_unit(const uint8_t* p, uint32_t off, uint32_t len) {
  if (off + 16u <= len && (reinterpret_cast<uintptr_t>(p) & 15u) == 0)
    return load_stream(p + off);
  const global_u8* g = gptr(p);
  uint32_t w[4] = {0, 0, 0, 0};
#pragma unroll
  for (int b = 0; b < 16; ++b)
    if (off + b < len) w[b >> 2] |= (uint32_t)g[off + b] << (8 * (b & 3));
  return make_uint4(w[0], w[1], w[2], w[3]);
}

// Store 16 parity bytes at byte offset off (byte stores if p is misaligned).
__device__ __forceinline__ void store_unit(uint8_t* p, uint32_t off, const uint4& v) {
  if ((reinterpret_cast<uintptr_t>(p) & 15u) == 0) {
    store_stream(p + off, v);
    return;
  }
  global_u8* g = gptr(p);
#pragma unroll
  for (int b = 0; b < 16; ++b) g[off + b] = (uint8_t)(word(v, b >> 2) >> (8 * (b & 3)));
}

// Store the bytes of v that fall below len at byte offset off of p.
__device__ __forceinline__ void store_unit_len(uint8_t* p, uint32_t off, uint32_t len,
                                               const uint4& v) {
  if (off + 16u <= len) {
    store_unit(p, off, v);
    return;
  }
  global_u8* g = gptr(p);
#pragma unroll
  for (int b = 0; b < 16; ++b)
    if (off + b < len) g[off + b] = (uint8_t)(word(v, b >> 2) >> (8 * (b & 3)));
}

template <int K, int M>
struct BatchArgs {
  const uint64_t* dptr;  // [n_stripes][K]
  const uint32_t* dlen;  // [n_stripes][K]
  const uint64_t* pptr;  // [n_stripes][M]
  const uint32_t* olen;  // [n_stripes][M] valid output bytes, or null = whole units
  const uint64_t* cptr;  // [n_stripes][K] copy of each data unit, zero-padded to
                         // unit_bytes (0 = no copy); read only when the kernel copies
  PermTab tab[M][K];
  uint32_t unit_bytes;
  uint32_t tiles_per_unit;   // tiles of kBlock*U*16 bytes in a unit
  uint32_t tiles_per_block;  // consecutive tiles one workgroup walks
  uint32_t blocks_per_unit;  // ceil(tiles_per_unit / tiles_per_block)
};

// 16 KiB of zeros in device memory, read-only: on the fast path a unit that
// ended before the current tile is read from here instead of branching, so
// the tile's k loads stay unconditional.  (Covers a tile of kBlock * U * 16
// bytes for U <= 4.)
__device__ __align__(16) uint8_t g_zero_tile[kBlock * 4 * 16] = {0};

// One tile of a stripe in which no unit ends strictly inside the tile and
// every output covers it (almost every tile).  src[j] points at the tile's
// first byte of unit j, or at g_zero_tile if the unit ended before the tile;
// dst[i] at the tile's first byte of output i.  (A branch around each store
// for outputs that ended early triples the register count, so such tiles
// take the edge path instead.)
//
// With COPY, cpy[j] points at the tile's first byte of unit j's copy (null:
// no copy) and the loaded chunk is stored there too: the data is read once
// for both the parity and the copy.
template <int K, int M, int U, bool COPY>
__device__ __forceinline__ void tile_full(const uint8_t* const (&src)[K], uint8_t* const (&dst)[M],
                                          uint8_t* const (&cpy)[K],
                                          const PermTab (&tab)[M][K]) {
  static_assert(kBlock * U * 16 <= sizeof(g_zero_tile), "tile larger than the zero tile");
  uint4 x[U][K];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const uint32_t rel = (u * kBlock + threadIdx.x) * 16u;
#pragma unroll
    for (int j = 0; j < K; ++j) x[u][j] = load_stream(src[j] + rel);
  }
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const uint32_t rel = (u * kBlock + threadIdx.x) * 16u;
    uint32_t acc[M][4] = {};
    gf_matvec16<K, M>(acc, x[u], tab);
#pragma unroll
    for (int i = 0; i < M; ++i)
      store_stream(dst[i] + rel, make_uint4(acc[i][0], acc[i][1], acc[i][2], acc[i][3]));
    if constexpr (COPY) {
#pragma unroll
      for (int j = 0; j < K; ++j)
        if (cpy[j]) store_stream(cpy[j] + rel, x[u][j]);
    }
  }
}

// A full tile whose units are not all 16-byte aligned (tensors that are
// views into a flat buffer at arbitrary offsets): one chunk per lane at a
// time, each unit read through load_realign (two aligned loads and a byte
// shift for a misaligned unit); the outputs are aligned.
template <int K, int M, int U, bool COPY>
__device__ __forceinline__ void tile_full_realign(const uint8_t* const (&src)[K],
                                                  uint8_t* const (&dst)[M],
                                                  uint8_t* const (&cpy)[K],
                                                  const PermTab (&tab)[M][K]) {
  constexpr int V = U >= 2 ? 2 : 1;  // chunks per lane in flight together
#pragma unroll 1
  for (int u0 = 0; u0 < U; u0 += V) {
    uint4 x[V][K];
#pragma unroll
    for (int v = 0; v < V; ++v) {
      const uint32_t rel = ((u0 + v) * kBlock + threadIdx.x) * 16u;
#pragma unroll
      for (int j = 0; j < K; ++j) x[v][j] = load_realign(src[j], rel);
    }
#pragma unroll
    for (int v = 0; v < V; ++v) {
      const uint32_t rel = ((u0 + v) * kBlock + threadIdx.x) * 16u;
      uint32_t acc[M][4] = {};
      gf_matvec16<K, M>(acc, x[v], tab);
#pragma unroll
      for (int i = 0; i < M; ++i)
        store_stream(dst[i] + rel, make_uint4(acc[i][0], acc[i][1], acc[i][2], acc[i][3]));
      if constexpr (COPY) {
#pragma unroll
        for (int j = 0; j < K; ++j)
          if (cpy[j]) store_stream(cpy[j] + rel, x[v][j]);
      }
    }
  }
}

// Any other tile (a unit or output ending inside it, an absent unit, a
// misaligned output): one unit at a time, descriptors re-read from memory,
// byte-granular at the ends.  Kept as a rolled loop so that its registers
// stay below the fast path's (the allocator takes the larger of the two).
//
// With COPY, each unit's chunk (zeros past its valid length) also goes to
// its copy, over the whole unit_bytes.
template <int K, int M, int U, bool COPY>
__device__ __forceinline__ void tile_edge(const BatchArgs<K, M>& a, uint32_t s, uint32_t base,
                                          const PermTab (&tab)[M][K]) {
  for (int u = 0; u < U; ++u) {
    const uint32_t off = (base + u * kBlock) * 16u;
    if (off >= a.unit_bytes) continue;
    uint32_t acc[M][4] = {};
#pragma unroll 1
    for (int j = 0; j < K; ++j) {
      const uint8_t* dj = reinterpret_cast<const uint8_t*>(a.dptr[(uint64_t)s * K + j]);
      uint32_t lj = dj ? a.dlen[(uint64_t)s * K + j] : 0u;
      lj = lj < a.unit_bytes ? lj : a.unit_bytes;
      uint4 xj = make_uint4(0u, 0u, 0u, 0u);
      if (off < lj) {
        xj = load_unit(dj, off, lj);
        Fields f[4];
#pragma unroll
        for (int dd = 0; dd < 4; ++dd) f[dd] = fields(word(xj, dd));
#pragma unroll
        for (int i = 0; i < M; ++i) {
          const PermTab t = tab[i][j];
#pragma unroll
          for (int dd = 0; dd < 4; ++dd) acc[i][dd] = mac1(acc[i][dd], t, f[dd]);
        }
      }
      if constexpr (COPY) {
        uint8_t* cj = reinterpret_cast<uint8_t*>(a.cptr[(uint64_t)s * K + j]);
        if (cj) store_unit(cj, off, xj);
      }
    }
#pragma unroll
    for (int i = 0; i < M; ++i) {
      uint8_t* pi = reinterpret_cast<uint8_t*>(a.pptr[(uint64_t)s * M + i]);
      uint32_t li = a.olen ? a.olen[(uint64_t)s * M + i] : a.unit_bytes;
      li = pi ? (li < a.unit_bytes ? li : a.unit_bytes) : 0u;
      if (off < li)
        store_unit_len(pi, off, li, make_uint4(acc[i][0], acc[i][1], acc[i][2], acc[i][3]));
    }
  }
}

template <int K, int M, int U, bool COPY>
__global__ void __launch_bounds__(kBlock) batched_kernel(const BatchArgs<K, M> a) {
  __shared__ PermTab tab[M][K];
  stage_tables<K, M>(tab, a.tab);
  // Workgroup b covers tiles [t0, t1) of one stripe: the descriptor loads and
  // table staging are paid once per span, not once per 4-8 KiB tile.
  const uint32_t s = blockIdx.x / a.blocks_per_unit;
  const uint32_t t0 = (blockIdx.x - s * a.blocks_per_unit) * a.tiles_per_block;
  const uint32_t t1 = min(t0 + a.tiles_per_block, a.tiles_per_unit);
  // Stripe-uniform facts (scalar registers): addresses, valid lengths, and
  // whether everything is 16-byte aligned.
  const uint8_t* d[K];
  uint32_t len[K];
  bool in_aligned = true, out_aligned = true;
#pragma unroll
  for (int j = 0; j < K; ++j) {
    d[j] = reinterpret_cast<const uint8_t*>(a.dptr[(uint64_t)s * K + j]);
    const uint32_t l = d[j] ? a.dlen[(uint64_t)s * K + j] : 0u;
    len[j] = l < a.unit_bytes ? l : a.unit_bytes;
    in_aligned &= (reinterpret_cast<uintptr_t>(d[j]) & 15u) == 0;
  }
  uint8_t* p[M];
  uint32_t olen[M];
#pragma unroll
  for (int i = 0; i < M; ++i) {
    p[i] = reinterpret_cast<uint8_t*>(a.pptr[(uint64_t)s * M + i]);
    const uint32_t l = p[i] ? (a.olen ? a.olen[(uint64_t)s * M + i] : a.unit_bytes) : 0u;
    olen[i] = l < a.unit_bytes ? l : a.unit_bytes;
    out_aligned &= (reinterpret_cast<uintptr_t>(p[i]) & 15u) == 0;
  }
  uint8_t* c[K];
#pragma unroll
  for (int j = 0; j < K; ++j) {
    c[j] = COPY ? reinterpret_cast<uint8_t*>(a.cptr[(uint64_t)s * K + j]) : nullptr;
    out_aligned &= (reinterpret_cast<uintptr_t>(c[j]) & 15u) == 0;
  }
  constexpr uint32_t kTileBytes = kBlock * U * 16u;
  for (uint32_t t = t0; t < t1; ++t) {
    const uint32_t base = t * (kBlock * U) + threadIdx.x;
    const uint32_t lo = t * kTileBytes, hi = lo + kTileBytes;
    // A tile is an edge tile when some unit ends strictly inside it or some
    // output does not cover it.
    const uint8_t* src[K];
    uint8_t* dst[M];
    uint8_t* cpy[K];
    bool edge = !out_aligned;
#pragma unroll
    for (int j = 0; j < K; ++j) {
      src[j] = len[j] >= hi ? d[j] + lo : g_zero_tile;
      edge |= len[j] > lo && len[j] < hi;
      cpy[j] = c[j] ? c[j] + lo : nullptr;
      if (COPY) edge |= c[j] && a.unit_bytes < hi;  // a copy always spans the unit
    }
#pragma unroll
    for (int i = 0; i < M; ++i) {
      dst[i] = p[i] + lo;
      edge |= olen[i] < hi;
    }
    if (edge)
      tile_edge<K, M, U, COPY>(a, s, base, tab);
    else if (in_aligned)
      tile_full<K, M, U, COPY>(src, dst, cpy, tab);
    else
      tile_full_realign<K, M, U, COPY>(src, dst, cpy, tab);
  }
}

template <int K, int M>
struct UpdateArgs {
  const uint64_t* nptr;  // [n_stripes][K], 0 = unit unchanged
  const uint64_t* optr;  // [n_stripes][K]
  const uint32_t* len;   // [n_stripes][K]
  const uint64_t* pptr;  // [n_stripes][M]
  PermTab tab[M][K];
  uint32_t unit_bytes;
  uint32_t tiles_per_unit;   // tiles of kBlock*16 bytes in a unit
  uint32_t tiles_per_block;  // consecutive tiles one workgroup walks
  uint32_t blocks_per_unit;
};

// Incremental update: each workgroup walks a span of tiles of one changed
// stripe.  The stripe's descriptors (which units changed, where their old
// and new bytes are, their lengths) are read once per span into scalar
// registers; a tile inside every changed unit, with everything 16-byte
// aligned, takes plain vector loads, any other tile the byte-granular path.
template <int K, int M>
__global__ void __launch_bounds__(kBlock) update_kernel(const UpdateArgs<K, M> a) {
  __shared__ PermTab tab[M][K];
  stage_tables<K, M>(tab, a.tab);
  const uint32_t s = blockIdx.x / a.blocks_per_unit;
  const uint32_t t0 = (blockIdx.x - s * a.blocks_per_unit) * a.tiles_per_block;
  const uint32_t t1 = min(t0 + a.tiles_per_block, a.tiles_per_unit);
  const uint8_t* nw[K];
  const uint8_t* od[K];
  uint32_t len[K];
  uint32_t full = a.unit_bytes;
  bool aligned = true, in_aligned = true;
#pragma unroll
  for (int j = 0; j < K; ++j) {
    nw[j] = reinterpret_cast<const uint8_t*>(a.nptr[(uint64_t)s * K + j]);
    od[j] = nw[j] ? reinterpret_cast<const uint8_t*>(a.optr[(uint64_t)s * K + j]) : nullptr;
    const uint32_t l = nw[j] ? a.len[(uint64_t)s * K + j] : 0u;
    len[j] = l < a.unit_bytes ? l : a.unit_bytes;
    if (nw[j]) {
      full = len[j] < full ? len[j] : full;
      in_aligned &=
          ((reinterpret_cast<uintptr_t>(nw[j]) | reinterpret_cast<uintptr_t>(od[j])) & 15u) == 0;
    }
  }
  // Misaligned units (views at arbitrary offsets) are realigned on the fast
  // path (load_realign); only the parity must be 16-byte aligned for it.  The
  // aligned case keeps plain loads: realigning every load cost the 1 %
  // update 5 % (0.338 -> 0.356 ms).
  uint8_t* p[M];
#pragma unroll
  for (int i = 0; i < M; ++i) {
    p[i] = reinterpret_cast<uint8_t*>(a.pptr[(uint64_t)s * M + i]);
    aligned &= (reinterpret_cast<uintptr_t>(p[i]) & 15u) == 0;
  }
  for (uint32_t t = t0; t < t1; ++t) {
    const uint32_t off = (t * kBlock + threadIdx.x) * 16u;
    if (off >= a.unit_bytes) continue;
    const bool fast = aligned && (t + 1) * (kBlock * 16u) <= full;
    uint32_t acc[M][4] = {};
    // The parity loads do not depend on the delta: issue them first so that
    // they are in flight together with the unit loads.
    uint4 pv[M];
    if (fast) {
#pragma unroll
      for (int i = 0; i < M; ++i) pv[i] = load_stream(p[i] + off);
    }
#pragma unroll
    for (int j = 0; j < K; ++j) {
      if (nw[j] == nullptr) continue;  // uniform: unchanged unit
      if (!fast && off >= len[j]) continue;
      uint4 vn, vo;
      if (fast && in_aligned) {
        vn = load_stream(nw[j] + off);
        vo = load_stream(od[j] + off);
      } else if (fast) {
        vn = load_realign(nw[j], off);
        vo = load_realign(od[j], off);
      } else {
        vn = load_unit(nw[j], off, len[j]);
        vo = load_unit(od[j], off, len[j]);
      }
      const uint4 dl = make_uint4(vn.x ^ vo.x, vn.y ^ vo.y, vn.z ^ vo.z, vn.w ^ vo.w);
      Fields f[4];
#pragma unroll
      for (int dd = 0; dd < 4; ++dd) f[dd] = fields(word(dl, dd));
#pragma unroll
      for (int i = 0; i < M; ++i) {
        asm volatile("" ::: "memory");
        const PermTab tj = tab[i][j];
#pragma unroll
        for (int dd = 0; dd < 4; ++dd) acc[i][dd] = mac1(acc[i][dd], tj, f[dd]);
      }
    }
#pragma unroll
    for (int i = 0; i < M; ++i) {
      const uint4 v = fast ? pv[i] : load_unit(p[i], off, a.unit_bytes);
      const uint4 w = make_uint4(v.x ^ acc[i][0], v.y ^ acc[i][1], v.z ^ acc[i][2], v.w ^ acc[i][3]);
      if (fast)
        store_stream(p[i] + off, w);
      else
        store_unit(p[i], off, w);
    }
  }
}

// --------------------------------------- batched kernels for wide codes --
// The batched encode/decode and the parity update for codes past the
// instantiated fast path (k > 16 or m > 4): k at run time, M a template
// parameter, one 16-byte chunk per lane (4 KiB tiles).  A workgroup stages
// its stripe's descriptors and the m x k tables in LDS; fast tiles issue the
// unit loads in groups of kWideGroup, edge tiles take the units one at a
// time with byte-granular ends, as in the fixed-size kernels.
constexpr uint32_t kWideTile = kBlock * 16u;

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
template <int M>
__device__ __forceinline__ bool stage_wide(WideStripe<M>& w, const BatchWideArgs& a, uint32_t s,
                                           bool update) {
  const int k = a.k;
  const uint32_t t = threadIdx.x;
  for (uint32_t i = t; i < (uint32_t)(M * k); i += kBlock) w.tab[i] = dev_perm_tab(a.coeff[i]);
  if (t < (uint32_t)k) {
    const uint8_t* d = reinterpret_cast<const uint8_t*>(a.dptr[(uint64_t)s * k + t]);
    const uint32_t l = d ? a.dlen[(uint64_t)s * k + t] : 0u;
    const uint8_t* o = update && d ? reinterpret_cast<const uint8_t*>(a.optr[(uint64_t)s * k + t])
                                   : nullptr;
    w.d[t] = d;
    w.o[t] = o;
    w.len[t] = l < a.unit_bytes ? l : a.unit_bytes;
  } else if (t >= 64 && t < 64 + M) {
    const uint32_t i = t - 64;
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

template <int M>
__global__ void __launch_bounds__(kBlock) batched_wide_kernel(const BatchWideArgs a) {
  __shared__ WideStripe<M> w;
  const uint32_t s = blockIdx.x / a.blocks_per_unit;
  const uint32_t t0 = (blockIdx.x - s * a.blocks_per_unit) * a.tiles_per_block;
  const uint32_t t1 = min(t0 + a.tiles_per_block, a.tiles_per_unit);
  const bool misaligned = stage_wide<M>(w, a, s, false);
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
template <int M>
__global__ void __launch_bounds__(kBlock) update_wide_kernel(const BatchWideArgs a) {
  __shared__ WideStripe<M> w;
  const uint32_t s = blockIdx.x / a.blocks_per_unit;
  const uint32_t t0 = (blockIdx.x - s * a.blocks_per_unit) * a.tiles_per_block;
  const uint32_t t1 = min(t0 + a.tiles_per_block, a.tiles_per_unit);
  stage_wide<M>(w, a, s, true);
  const int k = a.k;
  for (uint32_t t = t0; t < t1; ++t) {
    const uint32_t off = t * kWideTile + threadIdx.x * 16u;
    if (off >= a.unit_bytes) continue;
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

// ---------------------------------------------------------- host launch --

inline int hip_status() { return hipGetLastError() == hipSuccess ? EC_OK : EC_EHIP; }

// Grid for a grid-stride kernel over n16 chunks with U chunks per lane:
// enough workgroups to cover the range once, capped so a launch stays a few
// waves deep on 256 CUs.
inline unsigned grid_for(uint64_t n16, int U) {
  const uint64_t tiles = (n16 + (uint64_t)kBlock * U - 1) / ((uint64_t)kBlock * U);
  const uint64_t cap = 1u << 20;
  return (unsigned)(tiles < cap ? (tiles ? tiles : 1) : cap);
}

template <int K>
constexpr int unroll_for() {
  return K <= 8 ? 2 : 1;
}

// Chunks per lane of the batched launcher.  For k <= 8 a workgroup takes one
// 16 KiB tile per unit (U = 4, 222 VGPRs for RS(8,2), two waves per SIMD):
// fewer workgroups in flight means fewer stripes open at once, and this
// beat U = 2 with 16 KiB spans by 0-4 % (RS(8,2) over the 20.8 GB rank
// buffer in 4 MiB units 5.73 -> 5.86 TB/s of traffic; 1 MiB units 5.96 ->
// 6.19; RS(6,3) in 4 MiB units 5.81 -> 5.96; 64 KiB units 6.52 -> 6.67).
// Wider codes keep U = 1 (RS(12,4) ragged: U = 2 was 3 % slower).
template <int K>
constexpr int batched_unroll() {
  return K <= 8 ? 4 : 1;
}


template <int K, int M>
int launch_rs(const uint8_t* coeff, const uint8_t* const* d, uint8_t* const* o, uint64_t n16,
              hipStream_t st) {
  RsArgs<K, M> a;
  for (int j = 0; j < K; ++j) a.data[j] = d[j];
  for (int i = 0; i < M; ++i) a.out[i] = o[i];
  for (int i = 0; i < M; ++i)
    for (int j = 0; j < K; ++j) a.tab[i][j] = perm_tab(coeff[i * K + j]);
  a.n16 = n16;
  // One 16-byte chunk per lane per shard: with the two-window order this beat
  // two chunks by 2-6 % for k <= 8 (k > 8 needs U = 1 for registers anyway).
  constexpr int U = 1;
  hipLaunchKernelGGL((rs_kernel<K, M, U>), dim3(grid_for(n16, U)), dim3(kBlock), 0, st, a);
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
  hipLaunchKernelGGL((wide_kernel<M>), dim3(grid_for(n16, 1)), dim3(kBlock), 0, st, a);
  return hip_status();
}

template <int K>
int launch_xor(const uint8_t* const* d, uint8_t* o, uint64_t n16, hipStream_t st) {
  XorArgs<K> a;
  for (int j = 0; j < K; ++j) a.data[j] = d[j];
  a.out = o;
  a.n16 = n16;
  constexpr int U = unroll_for<K>();
  hipLaunchKernelGGL((xor_kernel<K, U>), dim3(grid_for(n16, U * (kXorBlock / kBlock))),
                     dim3(kXorBlock), 0, st, a);
  return hip_status();
}

template <int K, int M, int U, bool COPY>
int launch_batched_u(const uint8_t* coeff, const uint64_t* dptr, const uint32_t* dlen,
                     const uint64_t* pptr, const uint32_t* olen, const uint64_t* cptr,
                     uint32_t n_stripes, uint32_t unit_bytes, hipStream_t st) {
  BatchArgs<K, M> a;
  a.dptr = dptr;
  a.dlen = dlen;
  a.pptr = pptr;
  a.olen = olen;
  a.cptr = cptr;
  for (int i = 0; i < M; ++i)
    for (int j = 0; j < K; ++j) a.tab[i][j] = perm_tab(coeff[i * K + j]);
  const uint32_t unit16 = unit_bytes / 16u;
  a.unit_bytes = unit_bytes;
  a.tiles_per_unit = (unit16 + kBlock * U - 1) / (kBlock * U);
  // A workgroup walks up to span_bytes() of each unit (at least one tile),
  // keeping at least 2048 workgroups (8 per CU) in the launch.
  const uint32_t tile_bytes = kBlock * U * 16u;
  uint64_t tpb = span_bytes(unit_bytes) / tile_bytes;
  const uint64_t total_tiles = (uint64_t)n_stripes * a.tiles_per_unit;
  if (total_tiles / tpb < 2048) tpb = total_tiles / 2048;
  if (tpb < 1) tpb = 1;
  if (tpb > a.tiles_per_unit) tpb = a.tiles_per_unit;
  a.tiles_per_block = (uint32_t)tpb;
  a.blocks_per_unit = (a.tiles_per_unit + a.tiles_per_block - 1) / a.tiles_per_block;
  const uint64_t blocks = (uint64_t)n_stripes * a.blocks_per_unit;
  if (blocks > 0x7fffffffull) return EC_ERANGE;
  hipLaunchKernelGGL((batched_kernel<K, M, U, COPY>), dim3((unsigned)blocks), dim3(kBlock), 0,
                     st, a);
  return hip_status();
}

// The tile must not be larger than the units, or every tile holds a unit's
// end and takes the edge path: four chunks per lane (16 KiB tiles) only when
// the units are a multiple of 16 KiB, else one (4 KiB tiles).  RS(8,2) over
// 4 KiB units ran at 1.7 TB/s with 16 KiB tiles.
template <int K, int M>
int launch_batched(const uint8_t* coeff, const uint64_t* dptr, const uint32_t* dlen,
                   const uint64_t* pptr, const uint32_t* olen, uint32_t n_stripes,
                   uint32_t unit_bytes, hipStream_t st) {
  constexpr int U = batched_unroll<K>();
  if (U > 1 && unit_bytes % (kBlock * U * 16u) == 0)
    return launch_batched_u<K, M, U, false>(coeff, dptr, dlen, pptr, olen, nullptr, n_stripes,
                                            unit_bytes, st);
  return launch_batched_u<K, M, 1, false>(coeff, dptr, dlen, pptr, olen, nullptr, n_stripes,
                                          unit_bytes, st);
}

// Encode plus a zero-padded copy of every data unit (cptr), same tiling.
template <int K, int M>
int launch_batched_copy(const uint8_t* coeff, const uint64_t* dptr, const uint32_t* dlen,
                        const uint64_t* pptr, const uint64_t* cptr, uint32_t n_stripes,
                        uint32_t unit_bytes, hipStream_t st) {
  constexpr int U = batched_unroll<K>();
  if (U > 1 && unit_bytes % (kBlock * U * 16u) == 0)
    return launch_batched_u<K, M, U, true>(coeff, dptr, dlen, pptr, nullptr, cptr, n_stripes,
                                           unit_bytes, st);
  return launch_batched_u<K, M, 1, true>(coeff, dptr, dlen, pptr, nullptr, cptr, n_stripes,
                                         unit_bytes, st);
}

template <int K, int M>
int launch_update(const uint8_t* coeff, const uint64_t* nptr, const uint64_t* optr,
                  const uint32_t* len, const uint64_t* pptr, uint32_t n_stripes,
                  uint32_t unit_bytes, hipStream_t st) {
  UpdateArgs<K, M> a;
  a.nptr = nptr;
  a.optr = optr;
  a.len = len;
  a.pptr = pptr;
  for (int i = 0; i < M; ++i)
    for (int j = 0; j < K; ++j) a.tab[i][j] = perm_tab(coeff[i * K + j]);
  const uint32_t unit16 = unit_bytes / 16u;
  a.unit_bytes = unit_bytes;
  a.tiles_per_unit = (unit16 + kBlock - 1) / kBlock;
  // One tile per workgroup: each tile is a dependent chain (unit and parity
  // loads, then the parity store), so the update wants as many workgroups
  // in flight as it has tiles.  Measured for the 1 % update of 3,000 ragged
  // tensors in 64 KiB units (RS(12,4), 2,993 stripes): 3-tile spans 0.382 ms,
  // one tile 0.343 ms, one tile with the parity loads issued first 0.338 ms.
  // Spans grow only to keep the grid near 2^30 workgroups.
  const uint64_t total_tiles = (uint64_t)n_stripes * a.tiles_per_unit;
  uint64_t tpb = (total_tiles + 0x3fffffffull) >> 30;
  if (tpb < 1) tpb = 1;
  if (tpb > a.tiles_per_unit) tpb = a.tiles_per_unit;
  a.tiles_per_block = (uint32_t)tpb;
  a.blocks_per_unit = (a.tiles_per_unit + a.tiles_per_block - 1) / a.tiles_per_block;
  const uint64_t blocks = (uint64_t)n_stripes * a.blocks_per_unit;
  if (blocks > 0x7fffffffull) return EC_ERANGE;
  hipLaunchKernelGGL((update_kernel<K, M>), dim3((unsigned)blocks), dim3(kBlock), 0, st, a);
  return hip_status();
}

// Wide codes through the batched kernels: encode / decode (update = false,
// optr unused) or the parity update.  The same span rules as the fixed-size
// launchers: spans of span_bytes() with at least 2048 workgroups for the
// encode, one tile per workgroup for the update.
template <int M>
int launch_batched_wide(const uint8_t* coeff, int k, const uint64_t* dptr, const uint32_t* dlen,
                        const uint64_t* optr, const uint64_t* pptr, const uint32_t* olen,
                        uint32_t n_stripes, uint32_t unit_bytes, bool update, hipStream_t st) {
  BatchWideArgs a;
  a.dptr = dptr;
  a.dlen = dlen;
  a.optr = optr;
  a.pptr = pptr;
  a.olen = olen;
  for (int t = 0; t < M * k; ++t) a.coeff[t] = coeff[t];
  a.k = k;
  a.unit_bytes = unit_bytes;
  a.tiles_per_unit = (unit_bytes / 16u + kBlock - 1) / kBlock;
  const uint64_t total_tiles = (uint64_t)n_stripes * a.tiles_per_unit;
  uint64_t tpb = 1;
  if (!update) {
    tpb = span_bytes(unit_bytes) / kWideTile;
    if (total_tiles / tpb < 2048) tpb = total_tiles / 2048;
  } else {
    tpb = (total_tiles + 0x3fffffffull) >> 30;
  }
  if (tpb < 1) tpb = 1;
  if (tpb > a.tiles_per_unit) tpb = a.tiles_per_unit;
  a.tiles_per_block = (uint32_t)tpb;
  a.blocks_per_unit = (a.tiles_per_unit + a.tiles_per_block - 1) / a.tiles_per_block;
  const uint64_t blocks = (uint64_t)n_stripes * a.blocks_per_unit;
  if (blocks > 0x7fffffffull) return EC_ERANGE;
  if (update)
    hipLaunchKernelGGL((update_wide_kernel<M>), dim3((unsigned)blocks), dim3(kBlock), 0, st, a);
  else
    hipLaunchKernelGGL((batched_wide_kernel<M>), dim3((unsigned)blocks), dim3(kBlock), 0, st, a);
  return hip_status();
}

// Dispatch tables over the instantiated (K, M) grid.
using RsFn = int (*)(const uint8_t*, const uint8_t* const*, uint8_t* const*, uint64_t,
                     hipStream_t);
using XorFn = int (*)(const uint8_t* const*, uint8_t*, uint64_t, hipStream_t);
using BatchFn = int (*)(const uint8_t*, const uint64_t*, const uint32_t*, const uint64_t*,
                        const uint32_t*, uint32_t, uint32_t, hipStream_t);
using UpdFn = int (*)(const uint8_t*, const uint64_t*, const uint64_t*, const uint32_t*,
                      const uint64_t*, uint32_t, uint32_t, hipStream_t);

template <int K, int... Ms>
constexpr auto rs_row(std::integer_sequence<int, Ms...>) {
  return std::array<RsFn, sizeof...(Ms)>{&launch_rs<K, Ms + 1>...};
}
template <int... Ks>
constexpr auto rs_table(std::integer_sequence<int, Ks...>) {
  return std::array<std::array<RsFn, kFastMaxM>, sizeof...(Ks)>{
      rs_row<Ks + 1>(std::make_integer_sequence<int, kFastMaxM>{})...};
}
template <int K, int... Ms>
constexpr auto batch_row(std::integer_sequence<int, Ms...>) {
  return std::array<BatchFn, sizeof...(Ms)>{&launch_batched<K, Ms + 1>...};
}
template <int... Ks>
constexpr auto batch_table(std::integer_sequence<int, Ks...>) {
  return std::array<std::array<BatchFn, kFastMaxM>, sizeof...(Ks)>{
      batch_row<Ks + 1>(std::make_integer_sequence<int, kFastMaxM>{})...};
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
template <int K, int... Ms>
constexpr auto upd_row(std::integer_sequence<int, Ms...>) {
  return std::array<UpdFn, sizeof...(Ms)>{&launch_update<K, Ms + 1>...};
}
template <int... Ks>
constexpr auto upd_table(std::integer_sequence<int, Ks...>) {
  return std::array<std::array<UpdFn, kFastMaxM>, sizeof...(Ks)>{
      upd_row<Ks + 1>(std::make_integer_sequence<int, kFastMaxM>{})...};
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
const auto kBatchTable = batch_table(std::make_integer_sequence<int, kFastMaxK>{});
const auto kBatchCopyTable = batch_copy_table(std::make_integer_sequence<int, kFastMaxK>{});
const auto kUpdTable = upd_table(std::make_integer_sequence<int, kFastMaxK>{});
const auto kXorTable = xor_table(std::make_integer_sequence<int, kFastMaxK>{});
const auto kWideTable = wide_table(std::make_integer_sequence<int, EC_MAX_M>{});
using BatchWideFn = int (*)(const uint8_t*, int, const uint64_t*, const uint32_t*,
                            const uint64_t*, const uint64_t*, const uint32_t*, uint32_t, uint32_t,
                            bool, hipStream_t);
template <int... Ms>
constexpr auto batch_wide_table(std::integer_sequence<int, Ms...>) {
  return std::array<BatchWideFn, sizeof...(Ms)>{&launch_batched_wide<Ms + 1>...};
}
const auto kBatchWideTable = batch_wide_table(std::make_integer_sequence<int, EC_MAX_M>{});

inline bool fast_shape(int k, int m) { return k <= kFastMaxK && m <= kFastMaxM; }

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

int check_batch(const uint8_t* coeff, int k, int m, const void* a, const void* b,
                const void* c, uint32_t unit_bytes) {
  if (!coeff || !a || !b || !c || k < 1 || m < 1) return EC_EINVAL;
  if (k > EC_MAX_K || m > EC_MAX_M) return EC_ERANGE;
  if (unit_bytes == 0 || (unit_bytes & 15u)) return EC_EALIGN;
  // Byte offsets inside a unit are 32-bit in the kernels, with one tile of
  // headroom past the unit's end.
  if (unit_bytes > (1u << 31)) return EC_ERANGE;
  return EC_OK;
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

int ec_encode_batched(const uint8_t* coeff, int k, int m, const uint64_t* d_data_ptrs,
                      const uint32_t* d_data_len, const uint64_t* d_parity_ptrs,
                      uint32_t n_stripes, uint32_t unit_bytes, ec_stream_t stream) {
  int s = ec::check_batch(coeff, k, m, d_data_ptrs, d_data_len, d_parity_ptrs, unit_bytes);
  if (s != EC_OK) return s;
  if (n_stripes == 0) return EC_OK;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (!ec::fast_shape(k, m))
    return ec::kBatchWideTable[m - 1](coeff, k, d_data_ptrs, d_data_len, nullptr, d_parity_ptrs,
                                      nullptr, n_stripes, unit_bytes, false, st);
  return ec::kBatchTable[k - 1][m - 1](coeff, d_data_ptrs, d_data_len, d_parity_ptrs, nullptr,
                                       n_stripes, unit_bytes, st);
}

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
  s = ec::kBatchWideTable[m - 1](coeff, k, d_data_ptrs, d_data_len, nullptr, d_parity_ptrs,
                                 nullptr, n_stripes, unit_bytes, false, st);
  if (s != EC_OK) return s;
  const uint8_t one = 1;
  return ec::kBatchTable[0][0](&one, d_data_ptrs, d_data_len, d_copy_ptrs, nullptr,
                               (uint32_t)units, unit_bytes, st);
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
    return ec::kBatchWideTable[e - 1](rows, k, d_surv_ptrs, d_surv_len, nullptr, d_out_ptrs,
                                      d_out_len, n_stripes, unit_bytes, false, st);
  return ec::kBatchTable[k - 1][e - 1](rows, d_surv_ptrs, d_surv_len, d_out_ptrs, d_out_len,
                                       n_stripes, unit_bytes, st);
}

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
