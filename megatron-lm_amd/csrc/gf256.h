// gf256.h — host-side GF(2^8) algebra of the erasure-coding engine.
//
// Field GF(2^8) with reduction polynomial 0x11D and generator 0x02; the
// generator matrix is [I_k ; C] with C[i][j] = inv((k+i) ^ j).  The device
// kernels never see field elements directly: the host turns every
// coefficient c into the byte-permute tables of PermTab below.
#pragma once

#include <stdint.h>

namespace ec {

// c*x for a byte x, resolved with three v_perm_b32 byte selects:
//   c*x = T0[x & 7] ^ T1[(x >> 3) & 7] ^ T2[x >> 6]
// with T0[a] = c*a, T1[a] = c*(a << 3), T2[a] = c*(a << 6).  v_perm_b32 picks
// bytes out of a 64-bit pair, so an 8-entry table is one instruction; the
// byte is split 3+3+2 bits instead of the 4+4 of CPU split-nibble tables
// (a 16-entry table would cost two selects plus a blend per nibble).
// Bytes are packed little-endian: lo0 holds T0[0..3], hi0 T0[4..7].
struct PermTab {
  uint32_t lo0, hi0, lo1, hi1, t2;
};

uint8_t gf_mul(uint8_t a, uint8_t b);
uint8_t gf_inv(uint8_t a);
PermTab perm_tab(uint8_t c);

// Returns 0, or -3 when singular.
int gf_invert(const uint8_t* in, uint8_t* out, int n);

}  // namespace ec
