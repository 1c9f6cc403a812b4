// ec_device.h — device helpers shared by the gfx950 kernels of the C ABI
// (ec_flat.hip, ec_batched.hip, ec_batched_copy.hip, ec_update.hip).
//
// The work is byte-wise GF(2^8) arithmetic over HBM-resident shards: it is
// bound by HBM bandwidth, not by the matrix cores, so everything here is
// VALU code laid out for streaming.
//
// Data layout and mapping.
//   A shard is a flat byte range.  Lane l of a workgroup owns 16 bytes (one
//   global_load_dwordx4) of every shard at chunk index base + l, so each
//   wavefront reads 1 KiB contiguous per shard per load and the k loads of a
//   lane are all in flight together.  The m parity outputs of those bytes are
//   accumulated in VGPRs and written once: every input byte is read from HBM
//   exactly once and every parity byte written exactly once.  Loads and
//   stores are non-temporal (streamed past L2 and the Infinity Cache); some
//   kernels issue them as buffer instructions on a wave-uniform base
//   (load_wave, store_wave below).  The flat kernels run 64- or 128-lane
//   workgroups in launch order (flat_block in ec_flat.hip), the fixed-size
//   batched kernels and the update one-wavefront workgroups on 1 KiB tiles,
//   the kernels with k at run time 64- to 256-lane workgroups.  Measured on
//   MI355X for RS(6,3) over
//   256 MiB shards (HBM traffic): plain loads/stores and tables in SGPRs
//   5.48 TB/s; streaming access 5.90; plus LDS tables 6.15; 256-lane
//   workgroups streaming each shard at two places (even XCDs the first
//   half, odd XCDs the second) 5.9-6.5 depending on
//   the box and the buffer layout; one-wavefront workgroups in launch order
//   6.4 (see gf_matvec16 for the table-read order that keeps wider codes at
//   the same rate).
//
// GF multiply by a coefficient c (see PermTab in gf256.h): the byte x is cut
// into fields x[2:0], x[5:3], x[7:6]; each field indexes an 8- or 4-entry
// table of products held in one or two 32-bit registers, resolved for four
// bytes at once by one v_perm_b32.  The three partial products and the
// running parity are combined with v_bitop3_b32 (XOR3), so one coefficient
// costs 3 permutes + 1.5 XOR3 per dword, and the field selectors (5 ops per
// dword) are shared by all m outputs.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "ec_mi355.h"
#include "fastdiv.h"
#include "gf256.h"

namespace ec {

// Launchers shared between translation units.  batched_fast (ec_batched.hip)
// runs the fully unrolled batched kernel for k <= 16, m <= 4; batched_wide
// (ec_update.hip) the run-time-k kernels for any code up to EC_MAX_K x
// EC_MAX_M, as an encode/decode (update = false) or a parity update.
int batched_fast(int k, int m, const uint8_t* coeff, const uint64_t* dptr, const uint32_t* dlen,
                 const uint64_t* pptr, const uint32_t* olen, uint32_t n_stripes,
                 uint32_t unit_bytes, hipStream_t st);
int batched_wide(int m, const uint8_t* coeff, int k, const uint64_t* dptr, const uint32_t* dlen,
                 const uint64_t* optr, const uint64_t* pptr, const uint32_t* olen,
                 uint32_t n_stripes, uint32_t unit_bytes, bool update, hipStream_t st);

namespace {

constexpr int kBlock = 256;     // lanes per workgroup (4 wavefronts)
constexpr int kFastMaxK = 16;   // template-instantiated shard counts
constexpr int kFastMaxM = 4;
// Bytes of each unit a workgroup of the batched kernels for wide codes
// (batched_wide_kernel, 4 KiB tiles) walks: 8 KiB for units up to 256 KiB,
// 16 KiB above.  Measured on MI355X for the fixed-size batched kernel when it
// ran 256-lane workgroups (HBM traffic), spans of 64/32/16/8 KiB: RS(8,2)
// over 4 MiB units 5.31/5.50/5.71/5.54 TB/s; RS(8,2) over 64 KiB units
// 6.17/6.14/6.32/6.63; RS(12,4) over ragged 64 KiB units 5.87/5.86/6.13/6.22.
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

// The same accesses as buffer instructions on a wave-uniform base: the
// resource descriptor sits in SGPRs and each lane adds its byte offset
// (lane_off < 2^31).  The caller guarantees that base is the same for every
// lane of the wavefront (a kernel argument or descriptor entry plus a
// workgroup offset); a divergent base would not compile to one descriptor.
// Cache-policy bits of the buffer forms: 2 = nt (streaming), 16 = sc1.
// Measured on MI355X (HIP events, same box, loads and stores of the product
// kernels swapped one at a time): XOR(4) over 4 x 64 MiB 52.6 us with
// global nt loads and plain stores, 50.9 with sc1 buffer stores, 48.9 with
// nt buffer loads as well (4 x 256 MiB: 200.7 / 196.4 / 191.9).  The gain
// depends on the box: on one of eight it was nil.  Which kernel takes which
// form is stated at each kernel.
constexpr int kPolicyNt = 2;
constexpr int kPolicySc1 = 16;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t wave_rsrc(const void* base) {
  // dword 3 = 0x00020000: 32-bit data format, no swizzle, as gfx9 raw
  // buffers take it; num_records covers any lane offset below 2^31
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, 0x7fffffff, 0x00020000);
}

__device__ __forceinline__ uint4 load_wave(const void* base, uint32_t lane_off) {
  const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(wave_rsrc(base), lane_off, 0, kPolicyNt);
  return make_uint4(v.x, v.y, v.z, v.w);
}

template <int POLICY>
__device__ __forceinline__ void store_wave(void* base, uint32_t lane_off, const uint4& v) {
  const u32x4 w = {v.x, v.y, v.z, v.w};
  __builtin_amdgcn_raw_buffer_store_b128(w, wave_rsrc(base), lane_off, 0, POLICY);
}

// store_wave when keep, else nothing, without a branch: the descriptor's
// num_records is 0 when !keep, and the buffer unit's range check drops a
// store whose offset is at or past num_records before it reaches memory.
// keep must be wave-uniform, as base is.
template <int POLICY>
__device__ __forceinline__ void store_wave_if(void* base, uint32_t lane_off, const uint4& v,
                                              bool keep) {
  const u32x4 w = {v.x, v.y, v.z, v.w};
  const __amdgpu_buffer_rsrc_t r =
      __builtin_amdgcn_make_buffer_rsrc(base, 0, keep ? 0x7fffffff : 0, 0x00020000);
  __builtin_amdgcn_raw_buffer_store_b128(w, r, lane_off, 0, POLICY);
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
__device__ inline uint8_t dev_gf_mul(uint32_t a, uint32_t b) {
  uint32_t r = 0;
  for (int i = 0; i < 8; ++i) {
    if (b & 1u) r ^= a;
    b >>= 1;
    a <<= 1;
    if (a & 0x100u) a ^= 0x11Du;
  }
  return (uint8_t)r;
}

__device__ inline PermTab dev_perm_tab(uint32_t c) {
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

// ------------------------------------------------------- wide-code knobs --
// Codes past the instantiated fast path (k > 16 or m > 4, up to 32 x 16) on
// 16-byte-aligned shards: rs_kernel's column layout and launch order with
// the m outputs in registers (M is a template parameter) and k read at run time
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
// is the aligned dwordx4 load; otherwise one dwordx4 load at the unaligned
// address (the vector type below has alignment 1, so the compiler does not
// assume an alignment; for gfx950 it emits the single dwordx4 all the same,
// as it does for any 16-byte memcpy from a byte pointer, since the ROCm
// driver runs compute queues with unaligned memory access enabled),
// non-temporal like the aligned one.  It reads exactly the 16
// bytes asked for.  Measured on MI355X against the former form (the two
// aligned blocks holding the bytes, shifted into place with
// v_alignbyte_b32), HBM traffic, TB/s, one box: 600 fp32 tensor views of one
// flat buffer (6.82 GB, 450 of them misaligned) through the batched kernels,
// RS(12,4) in 64 KiB units 4.66 -> 5.88, RS(8,2) in 4 MiB units 3.51 ->
// 4.15, RS(6,3) in 1 MiB units 4.88 -> 5.94 (6.15-6.65 for aligned copies of
// the same tensors); RS(6,3) over six 64 MiB shards at skews 1-6 through the
// wide kernel 5.24 -> 5.62.  Aligned inputs do not take this path.
typedef uint32_t u32x4_unaligned __attribute__((ext_vector_type(4), aligned(1)));

__device__ __forceinline__ uint4 load_realign(const uint8_t* base, uint64_t off) {
  if ((reinterpret_cast<uintptr_t>(base) & 15u) == 0) return load_stream(base + off);
  const u32x4_unaligned v =
      __builtin_nontemporal_load(reinterpret_cast<const u32x4_unaligned*>(base + off));
  return make_uint4(v.x, v.y, v.z, v.w);
}

// ---------------------------------------------------------- unit access --
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

// ---------------------------------------------------------- host launch --

inline int hip_status() { return hipGetLastError() == hipSuccess ? EC_OK : EC_EHIP; }

// Grid for a grid-stride kernel over n16 chunks with U chunks per lane of a
// kBlock-lane workgroup: enough workgroups to cover the range once, capped so
// a launch stays a few waves deep on 256 CUs.
inline unsigned grid_for(uint64_t n16, int U) {
  const uint64_t tiles = (n16 + (uint64_t)kBlock * U - 1) / ((uint64_t)kBlock * U);
  const uint64_t cap = 1u << 20;
  return (unsigned)(tiles < cap ? (tiles ? tiles : 1) : cap);
}

// Grid of a grid-stride kernel with `lanes` lanes per workgroup and one chunk
// per lane: one workgroup per `lanes` chunks, up to 2^24 workgroups (shards
// up to 16 GiB with 64 lanes are covered in one pass).
inline unsigned grid_of(uint64_t n16, int lanes) {
  const uint64_t g = (n16 + (uint64_t)lanes - 1) / (uint64_t)lanes;
  const uint64_t cap = 1u << 24;
  return (unsigned)(g < cap ? (g ? g : 1) : cap);
}

// ----------------------------------------- grid order of batched launches --
// A batched launch codes n_spans spans (a span: consecutive tiles of one
// stripe, one workgroup each), stripe-major.  Units of kSliceMinUnit and
// more are walked in interleaved slices: with 2^s slices, workgroup b takes
// span (b mod 2^s) * slice_spans + b / 2^s, and the dispatcher deals
// consecutive workgroups to the 8 XCDs in turn, so the work in flight sits
// at 2^s unrelated offsets of the units instead of one (8 slices: each XCD
// streams its own eighth of the stripes).  With large units the units a
// workgroup reads lie a unit apart, and in launch order every workgroup in
// flight reads the same narrow band of offsets of them.  Measured on MI355X,
// fraction of the 8 TB/s roofline over one 20.8 GB buffer, single kernel,
// launch order / 2 / 4 / 8 slices, two boxes alike:
//   RS(12,4)  2 MiB 0.751 0.774 0.754 0.769    RS(6,3)  2 MiB 0.817 0.827 0.802 0.804
//   RS(12,4)  4 MiB 0.719 0.759 0.731 0.747    RS(6,3)  4 MiB 0.779 0.799 0.775 0.776
//   RS(12,4)  8 MiB 0.642 0.694 0.700 0.733    RS(6,3)  8 MiB 0.722 0.752 0.750 0.760
//   RS(12,4) 16 MiB 0.534 0.602 0.646 0.717    RS(8,2) 32 MiB 0.648 0.748 0.773 0.785
//   RS(12,4)  1 MiB 0.805 0.775 0.751 0.767 (launch order below 2 MiB)
//   RS(4,2)   4 MiB 0.817 0.823   -   0.789    RS(4,2)  2 MiB 0.839 0.849   -   0.827
// so an encode or decode over units of 2 MiB up to 8 MiB takes 2 slices and
// over larger ones 8.  The copying encode keeps 8 slices from 2 MiB up: its
// best order varied by code (RS(4,2) 4 MiB 0.744 0.715 - 0.726, RS(12,4)
// 4 MiB 0.645 0.672 - 0.754, RS(4,2) 2 MiB 0.776 0.781 - 0.772).  (Before
// the batched kernel's buffer accesses, 8 slices had measured best from
// 2 MiB up: RS(8,2) 2 MiB 0.741 -> 0.750, 4 MiB 0.723 -> 0.736, 8 MiB 0.691
// -> 0.736, 16 MiB 0.584 -> 0.700, 32 MiB 0.621 -> 0.720.)
constexpr uint32_t kSliceMinUnit = 2u << 20;
constexpr uint32_t kSliceWideUnit = 8u << 20;

struct SpanGrid {
  uint32_t n_spans;      // the spans to code
  uint32_t slice_shift;  // log2 of the interleaved slices (0: launch order)
  uint32_t slice_spans;  // ceil(n_spans / slices)
};

inline uint32_t slice_shift_for(uint32_t unit_bytes, bool copy) {
  if (unit_bytes < kSliceMinUnit) return 0u;
  return copy || unit_bytes >= kSliceWideUnit ? 3u : 1u;
}

// Fills g for `spans` (>= 1) spans in 2^shift slices and returns the grid,
// rounded up to whole slices; 0 when it exceeds 2^31 - 1 workgroups.
inline uint64_t span_grid(SpanGrid& g, uint64_t spans, uint32_t shift) {
  const uint64_t slices = 1ull << shift;
  if (spans + slices - 1 > 0x7fffffffull) return 0;
  g.n_spans = (uint32_t)spans;
  g.slice_shift = shift;
  g.slice_spans = (uint32_t)((spans + slices - 1) >> shift);
  return (uint64_t)g.slice_spans << shift;
}

// The span of this workgroup; n_spans or more for the few workgroups past
// the last span, which return before any work (uniform per workgroup).
// With shift 0 it is blockIdx.x; no branch, so the launch scalars load
// together.
__device__ __forceinline__ uint32_t span_of(const SpanGrid& g) {
  const uint32_t b = blockIdx.x;
  return (b & ((1u << g.slice_shift) - 1u)) * g.slice_spans + (b >> g.slice_shift);
}

inline bool fast_shape(int k, int m) { return k <= kFastMaxK && m <= kFastMaxM; }

inline int check_batch(const uint8_t* coeff, int k, int m, const void* a, const void* b,
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
