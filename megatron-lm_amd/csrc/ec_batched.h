// ec_batched.h — the fixed-size batched stripe kernel (batched_kernel), the
// two-kernel form for large RS(8,2) units (batched_full_kernel and
// batched_rest_kernel) and their launcher, shared by the plain encode/decode
// (ec_batched.hip) and the copying encode (ec_batched_copy.hip).
#pragma once

#include "ec_device.h"

namespace ec {
namespace {

// ------------------------------------------------ batched stripe kernels --
// One workgroup per span of tiles (n_stripes x blocks_per_unit spans),
// stripe-major: in launch order consecutive workgroups stream adjacent bytes
// of the same k units; units of kSliceMinUnit and more are dealt in 2 or 8
// interleaved slices instead (SpanGrid, slice_shift_for), except where the
// launcher splits the launch in two (RS(8,2), see split_pays).  The descriptor of a stripe is uniform
// across the workgroup (scalar loads).
//
// The product launches one-wavefront workgroups with one 16-byte chunk per
// lane, one 1 KiB tile of one stripe per workgroup (kBatchBlock, U = 1).
// Measured on MI355X (HBM traffic, GB/s) against the former launcher
// (256-lane workgroups walking 8-16 KiB of a stripe; four chunks per lane for
// k <= 8 and units that are a multiple of 16 KiB): config 5's RS(12,4) over
// 3,000 ragged tensors in 64 KiB units, encode 6271 -> 6316, copying encode
// 5440 -> 5791, decode of 4 positions 5559 -> 6124; RS(12,4) over 4 MiB
// units encode 5417 -> 5681, decode 5195 -> 5926; RS(6,3) over 1 MiB units
// encode 5999 -> 6651, decode 5844 -> 6424; RS(8,2) over 64 KiB units
// copying encode 5493 -> 6060, decode 6010 -> 6162, encode 6712 -> 6497; the
// 20.8 GB config 4 (RS(8,2), 4 MiB units) encode 5800 -> 5767.  Spans of
// 4 KiB per workgroup or 128-lane workgroups were in between.
constexpr int kBatchBlock = 64;

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
  uint32_t tiles_per_unit;   // tiles of B*U*16 bytes in a unit (B lanes)
  uint32_t tiles_per_block;  // consecutive tiles one workgroup walks
  uint32_t blocks_per_unit;  // ceil(tiles_per_unit / tiles_per_block)
  FastDiv by_blocks;         // division by blocks_per_unit
  SpanGrid grid;             // n_stripes * blocks_per_unit spans
  uint32_t rest_groups;      // workgroups per stripe of batched_rest_kernel
  FastDiv by_groups;         // division by rest_groups
};

// Zeros in device memory, read-only: on the fast path a unit that ended
// before the current tile is read from here instead of branching, so the
// tile's k loads stay unconditional.  (Covers a tile of B * U * 16 bytes for
// B * U <= 1024.)
__device__ __align__(16) uint8_t g_zero_tile[1024 * 16] = {0};

// Where tile_full's stores of outputs that ended before the tile point
// (their stores are dropped by the range check of store_wave_if, so nothing
// is written; a valid address all the same).
__device__ __align__(16) uint8_t g_sink_tile[1024 * 16];

// Store of 16 bytes at base + rel for tile_full (base wave-uniform); with
// WAVE a store with keep false is dropped (store_wave_if).
template <bool WAVE>
__device__ __forceinline__ void tile_store(uint8_t* base, uint32_t rel, const uint4& v,
                                           bool keep = true) {
  if constexpr (WAVE)
    store_wave_if<kPolicyNt | kPolicySc1>(base, rel, v, keep);
  else
    store_stream(base + rel, v);
}

// One tile of a stripe in which no unit ends strictly inside the tile
// (almost every tile).  src[j] points at the tile's first byte of unit j, or
// at g_zero_tile if the unit ended before the tile; dst[i] at the tile's
// first byte of output i.  Without WAVE every output covers the tile (a
// branch around each store for outputs that ended early triples the register
// count, so such tiles take the edge path).  With WAVE an output that ended
// at or before the tile's start (a short data unit rebuilt by a decode) has
// bit i of keep clear and its stores are dropped by the buffer range check:
// 1 % of config 5's decode tiles, which took the byte-granular edge path
// (same box, us per launch: lost data positions 0-3, 987 of them short,
// 4177 -> 4140; the bench's 1, 7, 12, 14 4326 -> 4333, unchanged within the
// noise).
//
// With COPY, cpy[j] points at the tile's first byte of unit j's copy (null:
// no copy) and the loaded chunk is stored there too: the data is read once
// for both the parity and the copy.
//
// WAVE selects the access forms.  The tile's addresses are wave-uniform, so
// with WAVE the loads are nt buffer loads and the stores nt+sc1 buffer
// stores on those bases (load_wave / store_wave); without, global nt loads
// and stores.  batched_kernel takes WAVE; batched_full_kernel and
// batched_rest_kernel do not.  Measured on MI355X (us per launch, global ->
// WAVE, same box): config 5 encode 4115 -> 4086, its decode of 4 positions
// 4413 -> 4341, its copying encode 7654 -> 7465; one 20.8 GB buffer through
// batched_kernel: RS(8,2) in 64 KiB units 3792 -> 3712, 1 MiB 3936 -> 3886,
// RS(12,4) 4 MiB 4625 -> 4608, 1 MiB 4415 -> 4372, RS(6,3) 1 MiB 4690 ->
// 4624, 4 MiB 5068 -> 5005.  batched_full_kernel (config 4) went the other
// way: 3934 -> 4358 with WAVE, 4029 with global loads and sc1 buffer stores.
template <int K, int M, int U, bool COPY, int B, bool WAVE>
__device__ __forceinline__ void tile_full(const uint8_t* const (&src)[K], uint8_t* const (&dst)[M],
                                          uint8_t* const (&cpy)[K],
                                          const PermTab (&tab)[M][K], uint32_t keep = ~0u) {
  static_assert(B * U * 16 <= sizeof(g_zero_tile), "tile larger than the zero tile");
  uint4 x[U][K];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const uint32_t rel = (u * B + threadIdx.x) * 16u;
#pragma unroll
    for (int j = 0; j < K; ++j)
      x[u][j] = WAVE ? load_wave(src[j], rel) : load_stream(src[j] + rel);
  }
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const uint32_t rel = (u * B + threadIdx.x) * 16u;
    uint32_t acc[M][4] = {};
    gf_matvec16<K, M>(acc, x[u], tab);
#pragma unroll
    for (int i = 0; i < M; ++i)
      tile_store<WAVE>(dst[i], rel, make_uint4(acc[i][0], acc[i][1], acc[i][2], acc[i][3]),
                       (keep >> i) & 1u);
    if constexpr (COPY) {
#pragma unroll
      for (int j = 0; j < K; ++j)
        if (cpy[j]) tile_store<WAVE>(cpy[j], rel, x[u][j]);
    }
  }
}

// A full tile whose units are not all 16-byte aligned (tensors that are
// views into a flat buffer at arbitrary offsets): one chunk per lane at a
// time, each unit read through load_realign (one unaligned dwordx4 load for
// a misaligned unit); the outputs are aligned.  A separate path from
// tile_full on purpose: routing misaligned units through tile_full itself
// (buffer loads at their byte addresses) changed the compiler's schedule of
// the aligned path, config 5's encode 4145 -> 4250 us.
template <int K, int M, int U, bool COPY, int B>
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
      const uint32_t rel = ((u0 + v) * B + threadIdx.x) * 16u;
#pragma unroll
      for (int j = 0; j < K; ++j) x[v][j] = load_realign(src[j], rel);
    }
#pragma unroll
    for (int v = 0; v < V; ++v) {
      const uint32_t rel = ((u0 + v) * B + threadIdx.x) * 16u;
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
template <int K, int M, int U, bool COPY, int B>
__device__ __forceinline__ void tile_edge(const BatchArgs<K, M>& a, uint32_t s, uint32_t base,
                                          const PermTab (&tab)[M][K]) {
  for (int u = 0; u < U; ++u) {
    const uint32_t off = (base + u * B) * 16u;
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

// A stripe's descriptors (uniform: scalar registers).  The arrays are dense
// ([n_stripes][K] / [n_stripes][M]), so every entry of the stripe is read
// unconditionally and the reads merge into a few wide scalar loads in flight
// together.  Reading a length only after its address had come back non-zero
// made every unit a dependent round trip: RS(8,2) over 4 MiB units then spent
// most of a one-tile workgroup's life in its preamble.
template <int K, int M, bool COPY>
struct StripeDesc {
  uint64_t dp[K], pp[M], cp[K];
  uint32_t dl[K], pl[M];
};

template <int K, int M, bool COPY>
__device__ __forceinline__ void read_stripe(StripeDesc<K, M, COPY>& r, const BatchArgs<K, M>& a,
                                            uint32_t s) {
#pragma unroll
  for (int j = 0; j < K; ++j) r.dp[j] = a.dptr[(uint64_t)s * K + j];
#pragma unroll
  for (int j = 0; j < K; ++j) r.dl[j] = a.dlen[(uint64_t)s * K + j];
#pragma unroll
  for (int i = 0; i < M; ++i) r.pp[i] = a.pptr[(uint64_t)s * M + i];
  if (a.olen) {
#pragma unroll
    for (int i = 0; i < M; ++i) r.pl[i] = a.olen[(uint64_t)s * M + i];
  } else {
#pragma unroll
    for (int i = 0; i < M; ++i) r.pl[i] = a.unit_bytes;
  }
#pragma unroll
  for (int j = 0; j < K; ++j) r.cp[j] = COPY ? a.cptr[(uint64_t)s * K + j] : 0u;
}

// Addresses, valid lengths (0 for an absent unit or output), and whether
// everything is 16-byte aligned.
template <int K, int M, bool COPY>
struct Stripe {
  const uint8_t* d[K];
  uint32_t len[K];
  uint8_t* p[M];
  uint32_t olen[M];
  uint8_t* c[K];
  bool in_aligned, out_aligned;
};

template <int K, int M, bool COPY>
__device__ __forceinline__ void stripe_facts(Stripe<K, M, COPY>& st,
                                             const StripeDesc<K, M, COPY>& r,
                                             uint32_t unit_bytes) {
  st.in_aligned = true;
  st.out_aligned = true;
#pragma unroll
  for (int j = 0; j < K; ++j) {
    st.d[j] = reinterpret_cast<const uint8_t*>(r.dp[j]);
    const uint32_t l = r.dp[j] ? r.dl[j] : 0u;
    st.len[j] = l < unit_bytes ? l : unit_bytes;
    st.in_aligned &= (r.dp[j] & 15u) == 0;
  }
#pragma unroll
  for (int i = 0; i < M; ++i) {
    st.p[i] = reinterpret_cast<uint8_t*>(r.pp[i]);
    const uint32_t l = r.pp[i] ? r.pl[i] : 0u;
    st.olen[i] = l < unit_bytes ? l : unit_bytes;
    st.out_aligned &= (r.pp[i] & 15u) == 0;
  }
#pragma unroll
  for (int j = 0; j < K; ++j) {
    st.c[j] = reinterpret_cast<uint8_t*>(r.cp[j]);
    st.out_aligned &= (r.cp[j] & 15u) == 0;
  }
}

// Tile t of stripe s through the path its contents need.  A tile is an edge
// tile when some unit ends strictly inside it or some output does not cover
// it (or an output is misaligned); a full tile with every unit aligned takes
// tile_full, one with misaligned units tile_full_realign.
template <int K, int M, int U, bool COPY, int B, bool WAVE>
__device__ __forceinline__ void code_tile(const BatchArgs<K, M>& a, uint32_t s, uint32_t t,
                                          const Stripe<K, M, COPY>& st,
                                          const PermTab (&tab)[M][K]) {
  constexpr uint32_t kTileBytes = B * U * 16u;
  const uint32_t base = t * (B * U) + threadIdx.x;
  const uint32_t lo = t * kTileBytes, hi = lo + kTileBytes;
  const uint8_t* src[K];
  uint8_t* dst[M];
  uint8_t* cpy[K];
  bool edge = !st.out_aligned;
#pragma unroll
  for (int j = 0; j < K; ++j) {
    src[j] = st.len[j] >= hi ? st.d[j] + lo : g_zero_tile;
    edge |= st.len[j] > lo && st.len[j] < hi;
    cpy[j] = st.c[j] ? st.c[j] + lo : nullptr;
    if (COPY) edge |= st.c[j] && a.unit_bytes < hi;  // a copy always spans the unit
  }
  // With WAVE an output that ended at or before lo is dropped from the full
  // path (keep); only an output ending strictly inside the tile makes it an
  // edge tile.  The realigning path has no dropped stores: there any output
  // short of hi makes an edge tile, as without WAVE.
  uint32_t keep = 0;
  bool short_out = false;
#pragma unroll
  for (int i = 0; i < M; ++i) {
    const bool covers = st.olen[i] >= hi;
    dst[i] = covers ? st.p[i] + lo : g_sink_tile;
    keep |= (uint32_t)covers << i;
    short_out |= !covers;
    edge |= st.olen[i] > lo && st.olen[i] < hi;
  }
  if (!WAVE || !st.in_aligned) edge |= short_out;
  if (edge)
    tile_edge<K, M, U, COPY, B>(a, s, base, tab);
  else if (st.in_aligned)
    tile_full<K, M, U, COPY, B, WAVE>(src, dst, cpy, tab, keep);
  else
    tile_full_realign<K, M, U, COPY, B>(src, dst, cpy, tab);
}

template <int K, int M, int U, bool COPY, int B>
__global__ void __launch_bounds__(B) batched_kernel(const BatchArgs<K, M> a) {
  // The span this workgroup takes (uniform: a scalar branch); the grid is
  // rounded up to whole slices, and the few workgroups past the last span
  // return before any work.
  const uint32_t b = span_of(a.grid);
  if (b >= a.grid.n_spans) return;
  // Workgroup b covers tiles [t0, t1) of one stripe: the descriptor loads and
  // table staging are paid once per span, not once per tile.
  const uint32_t s = fast_div(b, a.by_blocks);
  const uint32_t t0 = (b - s * a.blocks_per_unit) * a.tiles_per_block;
  const uint32_t t1 = min(t0 + a.tiles_per_block, a.tiles_per_unit);
  StripeDesc<K, M, COPY> r;
  read_stripe(r, a, s);
  __shared__ PermTab tab[M][K];
  stage_tables<K, M>(tab, a.tab);
  Stripe<K, M, COPY> st;
  stripe_facts(st, r, a.unit_bytes);
  for (uint32_t t = t0; t < t1; ++t) code_tile<K, M, U, COPY, B, true>(a, s, t, st, tab);
}

// ---- large units: the full tiles and the rest, as two kernels ----------
// For RS(8,2) over units of kSplitMinUnit up to kSplitMaxUnit (not for the
// copying encode) a launch is two kernels over disjoint tiles of every
// stripe:
//  - batched_full_kernel, one workgroup per tile in launch order, codes the
//    tiles of an aligned stripe that hold no unit end strictly inside them,
//    as far as every output covers them (vector_end, end_inside), and
//    returns at once on the others: nothing but the vector path, and the
//    compiler spreads its unit loads between the GF arithmetic;
//  - batched_rest_kernel, rest_groups workgroups per stripe, codes the other
//    tiles through code_tile: at most k tiles holding a unit end, and the
//    tiles some output does not cover.  A stripe of whole units (a rank's
//    buffer cut into units: every stripe but the last) returns after reading
//    its descriptors.
// Measured on MI355X over 20.8 GB of data, fraction of the 8 TB/s roofline
// at 2 / 4 / 8 MiB units, the single kernel (8 slices) -> the two kernels,
// each pair from one box:
//   RS(8,2)   0.785 0.763 0.762 -> 0.831 0.818 0.787
//   RS(8,1)   0.759 0.745 0.742 -> 0.760 0.733 0.686
//   RS(6,2)   0.791 0.773 0.774 -> 0.817 0.788 0.753
//   RS(4,2)   0.831 0.800 0.797 -> 0.833 0.805 0.782
//   RS(4,1)   0.809 0.796 0.779 -> 0.806 0.790 0.779
//   RS(6,3)   0.817 0.795 0.785 -> 0.781 0.763 0.725
//   RS(10,2)  0.776 0.750 0.752 -> 0.723 0.720 0.695
//   RS(16,1)  0.748 0.736 0.739 -> 0.709 0.666 0.628
//   RS(5,4)   0.742 0.723 0.716 -> 0.612 0.611 0.591
// so only RS(8,2), the code of a rank's checkpoint buffer and the one code
// that gains at every size, takes the split (split_pays).  Below 2 MiB its single kernel runs in launch order at
// 0.82-0.85 and the split gains nothing; at 16 and 32 MiB the split lost
// (0.662 against 0.714, 0.668 against 0.772).
constexpr uint32_t kSplitMinUnit = 2u << 20;
constexpr uint32_t kSplitMaxUnit = 16u << 20;

template <int K, int M>
constexpr bool split_pays() {
  return K == 8 && M == 2;
}

// Which tiles of a stripe the vector kernel codes: an aligned stripe's tiles
// below out_end (from out_end on some output does not cover the tile: output
// i covers tile t iff olen[i] >= (t + 1) * kTileBytes) that hold no unit end
// strictly inside them (every unit covers such a tile or ended before it,
// and reads as zeros there).  batched_rest_kernel codes the others: the at
// most K tiles below out_end that hold a unit end, then [out_end, tiles);
// out_end is 0 for a stripe with a misaligned address, whose tiles all go
// to the rest kernel.
template <int K, int M, bool COPY>
__device__ __forceinline__ uint32_t vector_end(const Stripe<K, M, COPY>& st, uint32_t tiles,
                                               uint32_t tile_bytes) {
  uint32_t out_end = tiles;
#pragma unroll
  for (int i = 0; i < M; ++i) {
    const uint32_t t = st.olen[i] / tile_bytes;
    out_end = t < out_end ? t : out_end;
  }
  return st.in_aligned && st.out_aligned ? out_end : 0u;
}

// Whether a unit of the stripe ends strictly inside tile t.
template <int K, int M, bool COPY>
__device__ __forceinline__ bool end_inside(const Stripe<K, M, COPY>& st, uint32_t t,
                                           uint32_t tile_bytes) {
  const uint32_t lo = t * tile_bytes, hi = lo + tile_bytes;
  bool e = false;
#pragma unroll
  for (int j = 0; j < K; ++j) e |= st.len[j] > lo && st.len[j] < hi;
  return e;
}

// Unit j's end tile when it ends strictly inside a tile below out_end and no
// unit before it ends in the same tile (so that each end tile is listed
// once); else tiles (none).
template <int K, int M, bool COPY>
__device__ __forceinline__ uint32_t first_end_tile(const Stripe<K, M, COPY>& st, int j,
                                                   uint32_t out_end, uint32_t tiles,
                                                   uint32_t tile_bytes) {
  const uint32_t t = st.len[j] / tile_bytes;
  if (st.len[j] % tile_bytes == 0 || t >= out_end) return tiles;
#pragma unroll
  for (int q = 0; q < K; ++q)
    if (q < j && st.len[q] % tile_bytes != 0 && st.len[q] / tile_bytes == t) return tiles;
  return t;
}

template <int K, int M, int B>
__global__ void __launch_bounds__(B) batched_full_kernel(const BatchArgs<K, M> a) {
  // One tile per workgroup (the launcher splits only when tiles_per_block
  // is 1).
  const uint32_t b = span_of(a.grid);
  if (b >= a.grid.n_spans) return;
  const uint32_t s = fast_div(b, a.by_blocks);
  const uint32_t t = b - s * a.blocks_per_unit;
  StripeDesc<K, M, false> r;
  read_stripe(r, a, s);
  __shared__ PermTab tab[M][K];
  stage_tables<K, M>(tab, a.tab);
  Stripe<K, M, false> st;
  stripe_facts(st, r, a.unit_bytes);
  constexpr uint32_t kTileBytes = B * 16u;
  const bool mine = t < vector_end(st, a.tiles_per_unit, kTileBytes) &&
                    !end_inside(st, t, kTileBytes);
  // A loop of zero or one tile rather than a return and straight-line code:
  // in this form the compiler interleaves the unit loads with the GF
  // arithmetic (RS(8,2): 122 VGPRs against 142 with the loads hoisted), and
  // RS(8,2) over 4 MiB units runs at 0.82 of the roofline against 0.79.
  const uint32_t t_end = mine ? t + 1 : t;
  if (t >= t_end) return;   // the rest kernel's
  for (uint32_t u = t; u < t_end; ++u) {
    const uint32_t lo = u * kTileBytes, hi = lo + kTileBytes;
    const uint8_t* src[K];
    uint8_t* dst[M];
    uint8_t* cpy[K];
#pragma unroll
    for (int j = 0; j < K; ++j) {
      src[j] = st.len[j] >= hi ? st.d[j] + lo : g_zero_tile;
      cpy[j] = nullptr;
    }
#pragma unroll
    for (int i = 0; i < M; ++i) dst[i] = st.p[i] + lo;
    tile_full<K, M, 1, false, B, false>(src, dst, cpy, tab);
  }
}

template <int K, int M, int B>
__global__ void __launch_bounds__(B) batched_rest_kernel(const BatchArgs<K, M> a) {
  const uint32_t s = fast_div(blockIdx.x, a.by_groups);
  const uint32_t g = blockIdx.x - s * a.rest_groups;
  StripeDesc<K, M, false> r;
  read_stripe(r, a, s);
  Stripe<K, M, false> st;
  stripe_facts(st, r, a.unit_bytes);
  constexpr uint32_t kTileBytes = B * 16u;
  const uint32_t tiles = a.tiles_per_unit;
  const uint32_t out_end = vector_end(st, tiles, kTileBytes);
  // The tiles batched_full_kernel leaves: the distinct end tiles below
  // out_end (at most K), then [out_end, tiles), numbered in that order and
  // dealt round robin to the stripe's workgroups.
  uint32_t ends = 0;
#pragma unroll
  for (int j = 0; j < K; ++j) ends += first_end_tile(st, j, out_end, tiles, kTileBytes) < tiles;
  const uint32_t total = ends + (tiles - out_end);
  if (g >= total) return;
  __shared__ PermTab tab[M][K];
  stage_tables<K, M>(tab, a.tab);
  for (uint32_t n = g; n < total; n += a.rest_groups) {
    uint32_t t = out_end + (n - ends);
    if (n < ends) {   // the n-th distinct end tile, in unit order
      uint32_t c = 0;
#pragma unroll
      for (int j = 0; j < K; ++j) {
        const uint32_t e = first_end_tile(st, j, out_end, tiles, kTileBytes);
        if (e < tiles) {
          if (c == n) t = e;
          ++c;
        }
      }
    }
    code_tile<K, M, 1, false, B, false>(a, s, t, st, tab);
  }
}

template <int K, int M, int U, bool COPY, int B>
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
  a.tiles_per_unit = (unit16 + B * U - 1) / (B * U);
  // One tile per workgroup; spans of consecutive tiles only to keep the grid
  // below 2^30 workgroups.
  const uint64_t total_tiles = (uint64_t)n_stripes * a.tiles_per_unit;
  uint64_t tpb = (total_tiles + 0x3fffffffull) >> 30;
  if (tpb < 1) tpb = 1;
  if (tpb > a.tiles_per_unit) tpb = a.tiles_per_unit;
  a.tiles_per_block = (uint32_t)tpb;
  a.blocks_per_unit = (a.tiles_per_unit + a.tiles_per_block - 1) / a.tiles_per_block;
  a.by_blocks = make_fastdiv(a.blocks_per_unit);
  const bool split = !COPY && U == 1 && split_pays<K, M>() && a.tiles_per_block == 1 &&
                     unit_bytes >= kSplitMinUnit && unit_bytes < kSplitMaxUnit;
  const uint64_t blocks = span_grid(a.grid, (uint64_t)n_stripes * a.blocks_per_unit,
                                    split ? 0u : slice_shift_for(unit_bytes, COPY));
  if (blocks == 0) return EC_ERANGE;
  if constexpr (!COPY && U == 1 && split_pays<K, M>()) {
    if (split) {
      // Enough rest workgroups to fill the chip when whole stripes are
      // misaligned (about 8192 in all), at most one per tile.
      uint64_t groups = (8192u + (uint64_t)n_stripes - 1) / n_stripes;
      if (groups > a.tiles_per_unit) groups = a.tiles_per_unit;
      a.rest_groups = (uint32_t)groups;
      a.by_groups = make_fastdiv(a.rest_groups);
      const uint64_t rest_blocks = (uint64_t)n_stripes * groups;
      if (rest_blocks > 0x7fffffffull) return EC_ERANGE;
      hipLaunchKernelGGL((batched_full_kernel<K, M, B>), dim3((unsigned)blocks), dim3(B), 0,
                         st, a);
      hipLaunchKernelGGL((batched_rest_kernel<K, M, B>), dim3((unsigned)rest_blocks),
                         dim3(B), 0, st, a);
      return hip_status();
    }
  }
  hipLaunchKernelGGL((batched_kernel<K, M, U, COPY, B>), dim3((unsigned)blocks), dim3(B), 0,
                     st, a);
  return hip_status();
}

}  // namespace
}  // namespace ec
