// ec_update.h — the incremental parity update for k <= 16, m <= 4
// (update_kernel) and its launcher, used by ec_parity_update (ec_update.hip).
//
//   parity_i ^= XOR_j C[i][j] * (new_j ^ old_j)
//
// over the changed units j of each listed stripe.  Per changed byte the
// update reads new, old and the m parity bytes and writes the m parity bytes
// back: a read-modify-write stream in which the parity dominates (with one
// changed unit of 12 per RS(12,4) stripe, 8 of every 10 bytes moved are
// parity).
#pragma once

#include "ec_device.h"

namespace ec {
namespace {

template <int K, int M>
struct UpdateArgs {
  const uint64_t* nptr;  // [n_stripes][K], 0 = unit unchanged
  const uint64_t* optr;  // [n_stripes][K]
  const uint32_t* len;   // [n_stripes][K]
  const uint64_t* pptr;  // [n_stripes][M]
  PermTab tab[M][K];
  uint32_t unit_bytes;
  uint32_t tiles_per_unit;   // tiles of B*U*16 bytes in a unit (B lanes, U chunks each)
  uint32_t tiles_per_block;  // consecutive tiles one workgroup walks
  uint32_t blocks_per_unit;  // ceil(tiles_per_unit / tiles_per_block)
  FastDiv by_blocks;         // division by blocks_per_unit
  SpanGrid grid;             // n_stripes * blocks_per_unit spans
};

// Each workgroup walks a span of tiles of one changed stripe (one tile,
// unless the grid would pass 2^30 workgroups).  The stripe's descriptors
// (which units changed, where their old and new bytes are, their lengths)
// are read once per span into scalar registers, every entry unconditionally
// (the arrays are dense) so that the reads merge into wide scalar loads in
// flight together rather than one dependent round trip per unit.
//
// A tile inside every changed unit, with the parity 16-byte aligned, takes
// the vector path: lane l owns the U chunks l, l + B, ... of the tile; the
// parity loads of all U chunks are issued first (they do not depend on the
// delta), then each changed unit's new and old chunks, so a lane has
// U * (M + 2) loads in flight.  Misaligned units (views at arbitrary
// offsets) are realigned there (load_realign); the aligned case keeps plain
// loads (realigning every load cost the 1 % update 5 %).  The parity
// stores are nt+sc1 buffer stores on the tile's wave-uniform base
// (store_wave): config 5's 1 % update 310.9 -> 304.9 us against global nt
// stores, same box; buffer loads as well measured 312.6.  Any other tile
// takes the byte-granular path one chunk at a time.  Parity chunks that
// start at or past the end of the stripe's longest changed unit are neither
// read nor written: the delta is zero there.
template <int K, int M, int B, int U>
__global__ void __launch_bounds__(B) update_kernel(const UpdateArgs<K, M> a) {
  const uint32_t b = span_of(a.grid);
  if (b >= a.grid.n_spans) return;
  const uint32_t s = fast_div(b, a.by_blocks);
  const uint32_t t0 = (b - s * a.blocks_per_unit) * a.tiles_per_block;
  const uint32_t t1 = min(t0 + a.tiles_per_block, a.tiles_per_unit);
  uint64_t np[K], op[K];
  uint32_t nl[K];
#pragma unroll
  for (int j = 0; j < K; ++j) np[j] = a.nptr[(uint64_t)s * K + j];
#pragma unroll
  for (int j = 0; j < K; ++j) op[j] = a.optr[(uint64_t)s * K + j];
#pragma unroll
  for (int j = 0; j < K; ++j) nl[j] = a.len[(uint64_t)s * K + j];
  __shared__ PermTab tab[M][K];
  stage_tables<K, M>(tab, a.tab);
  const uint8_t* nw[K];
  const uint8_t* od[K];
  uint32_t len[K];
  uint32_t full = a.unit_bytes;   // shortest changed unit
  uint32_t longest = 0;           // longest changed unit: past it the delta is zero
  bool aligned = true, in_aligned = true;
#pragma unroll
  for (int j = 0; j < K; ++j) {
    nw[j] = reinterpret_cast<const uint8_t*>(np[j]);
    od[j] = np[j] ? reinterpret_cast<const uint8_t*>(op[j]) : nullptr;
    const uint32_t l = np[j] ? nl[j] : 0u;
    len[j] = l < a.unit_bytes ? l : a.unit_bytes;
    if (nw[j]) {
      full = len[j] < full ? len[j] : full;
      longest = len[j] > longest ? len[j] : longest;
      in_aligned &=
          ((reinterpret_cast<uintptr_t>(nw[j]) | reinterpret_cast<uintptr_t>(od[j])) & 15u) == 0;
    }
  }
  uint8_t* p[M];
#pragma unroll
  for (int i = 0; i < M; ++i) {
    p[i] = reinterpret_cast<uint8_t*>(a.pptr[(uint64_t)s * M + i]);
    aligned &= (reinterpret_cast<uintptr_t>(p[i]) & 15u) == 0;
  }
  constexpr uint32_t kTile = B * U * 16u;
  for (uint32_t t = t0; t < t1; ++t) {
    const uint32_t lo = t * kTile;
    if (lo >= longest) break;   // uniform: no changed byte from here on
    if (aligned && lo + kTile <= full) {
      uint4 pv[U][M];
#pragma unroll
      for (int u = 0; u < U; ++u)
#pragma unroll
        for (int i = 0; i < M; ++i) pv[u][i] = load_stream(p[i] + lo + (u * B + threadIdx.x) * 16u);
      uint32_t acc[U][M][4] = {};
#pragma unroll
      for (int j = 0; j < K; ++j) {
        if (nw[j] == nullptr) continue;  // uniform: unchanged unit
        uint4 vn[U], vo[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const uint32_t rel = (u * B + threadIdx.x) * 16u;
          const uint32_t off = lo + rel;
          if (in_aligned) {
            // (base + lo) is wave-uniform: a scalar base and a 32-bit lane
            // offset per load, not a 64-bit address per lane (same box:
            // config 5's update 306.9 -> 303.9 us)
            vn[u] = load_stream(nw[j] + lo + rel);
            vo[u] = load_stream(od[j] + lo + rel);
          } else {
            vn[u] = load_realign(nw[j], off);
            vo[u] = load_realign(od[j], off);
          }
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const uint4 dl =
              make_uint4(vn[u].x ^ vo[u].x, vn[u].y ^ vo[u].y, vn[u].z ^ vo[u].z, vn[u].w ^ vo[u].w);
          Fields f[4];
#pragma unroll
          for (int dd = 0; dd < 4; ++dd) f[dd] = fields(word(dl, dd));
#pragma unroll
          for (int i = 0; i < M; ++i) {
            asm volatile("" ::: "memory");
            const PermTab tj = tab[i][j];
#pragma unroll
            for (int dd = 0; dd < 4; ++dd) acc[u][i][dd] = mac1(acc[u][i][dd], tj, f[dd]);
          }
        }
      }
#pragma unroll
      for (int u = 0; u < U; ++u)
#pragma unroll
        for (int i = 0; i < M; ++i)
          store_wave<kPolicyNt | kPolicySc1>(
              p[i] + lo, (u * B + threadIdx.x) * 16u,
              make_uint4(pv[u][i].x ^ acc[u][i][0], pv[u][i].y ^ acc[u][i][1],
                         pv[u][i].z ^ acc[u][i][2], pv[u][i].w ^ acc[u][i][3]));
      continue;
    }
    // edge tile: a changed unit ends inside it or before it, or the parity
    // is misaligned; parity bytes past the longest changed unit stay as they are
#pragma unroll 1
    for (int u = 0; u < U; ++u) {
      const uint32_t off = lo + (u * B + threadIdx.x) * 16u;
      if (off >= longest) continue;
      uint32_t acc[M][4] = {};
#pragma unroll
      for (int j = 0; j < K; ++j) {
        if (nw[j] == nullptr || off >= len[j]) continue;
        const uint4 vn = load_unit(nw[j], off, len[j]);
        const uint4 vo = load_unit(od[j], off, len[j]);
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
        const uint4 v = load_unit(p[i], off, a.unit_bytes);
        store_unit(p[i], off, make_uint4(v.x ^ acc[i][0], v.y ^ acc[i][1], v.z ^ acc[i][2],
                                         v.w ^ acc[i][3]));
      }
    }
  }
}

// One launch of update_kernel<K, M, B, U> over n_stripes stripes, the spans
// in launch order (slice_shift 0) or in 2^slice_shift interleaved slices
// (SpanGrid).  One tile per workgroup: each tile is a dependent chain (unit
// and parity loads, then the parity store), so the update wants as many
// workgroups in flight as it has tiles; spans of several tiles only keep the
// grid below 2^30 workgroups.
template <int K, int M, int B, int U>
int launch_update(const uint8_t* coeff, const uint64_t* nptr, const uint64_t* optr,
                  const uint32_t* len, const uint64_t* pptr, uint32_t n_stripes,
                  uint32_t unit_bytes, uint32_t slice_shift, hipStream_t st) {
  static_assert(B >= M * K, "stage_tables needs a lane per table");
  UpdateArgs<K, M> a;
  a.nptr = nptr;
  a.optr = optr;
  a.len = len;
  a.pptr = pptr;
  for (int i = 0; i < M; ++i)
    for (int j = 0; j < K; ++j) a.tab[i][j] = perm_tab(coeff[i * K + j]);
  const uint32_t unit16 = unit_bytes / 16u;
  a.unit_bytes = unit_bytes;
  a.tiles_per_unit = (unit16 + B * U - 1) / (B * U);
  const uint64_t total_tiles = (uint64_t)n_stripes * a.tiles_per_unit;
  uint64_t tpb = (total_tiles + 0x3fffffffull) >> 30;
  if (tpb < 1) tpb = 1;
  if (tpb > a.tiles_per_unit) tpb = a.tiles_per_unit;
  a.tiles_per_block = (uint32_t)tpb;
  a.blocks_per_unit = (a.tiles_per_unit + a.tiles_per_block - 1) / a.tiles_per_block;
  a.by_blocks = make_fastdiv(a.blocks_per_unit);
  const uint64_t blocks =
      span_grid(a.grid, (uint64_t)n_stripes * a.blocks_per_unit, slice_shift);
  if (blocks == 0) return EC_ERANGE;
  hipLaunchKernelGGL((update_kernel<K, M, B, U>), dim3((unsigned)blocks), dim3(B), 0, st, a);
  return hip_status();
}

}  // namespace
}  // namespace ec
