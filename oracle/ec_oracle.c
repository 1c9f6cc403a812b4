/*
 * ec_oracle.c — scalar CPU oracle of the erasure-coding hot path.
 *
 * TEST INFRASTRUCTURE: loaded only by tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg, as the checker.  The reference contains no
 * erasure coder (nothing to cite for the arithmetic); every function is
 * restated from the mathematics, and the conventions are listed in
 * ec_oracle.h.  Written for clarity, not speed: byte loops and a product
 * table built from the bitwise multiply.
 */
#include "ec_oracle.h"

#include <stdlib.h>
#include <string.h>

#define POLY 0x11Du

/* Carry-less ("Russian peasant") multiply with reduction by 0x11D. */
uint8_t ecref_gf_mul(uint8_t a, uint8_t b) {
  unsigned x = a, y = b, r = 0;
  while (y) {
    if (y & 1u) r ^= x;
    y >>= 1;
    x <<= 1;
    if (x & 0x100u) x ^= POLY;
  }
  return (uint8_t)r;
}

/* a^254 = a^-1 for a != 0 (the multiplicative group has order 255). */
uint8_t ecref_gf_inv(uint8_t a) {
  if (a == 0) return 0;
  uint8_t r = 1;
  for (int i = 0; i < 254; ++i) r = ecref_gf_mul(r, a);
  return r;
}

int ecref_cauchy(int k, int m, uint8_t* out) {
  if (k < 1 || m < 1 || k + m > 256) return -1;
  for (int i = 0; i < m; ++i)
    for (int j = 0; j < k; ++j)
      out[i * k + j] = ecref_gf_inv((uint8_t)((k + i) ^ j));
  return 0;
}

/* Gauss-Jordan elimination on [A | I]; pivot = first non-zero below. */
int ecref_gf_invert(const uint8_t* in, uint8_t* out, int n) {
  if (n < 1) return -1;
  uint8_t* a = (uint8_t*)malloc((size_t)n * n);
  memcpy(a, in, (size_t)n * n);
  memset(out, 0, (size_t)n * n);
  for (int i = 0; i < n; ++i) out[i * n + i] = 1;
  for (int c = 0; c < n; ++c) {
    int p = c;
    while (p < n && a[p * n + c] == 0) ++p;
    if (p == n) {
      free(a);
      return -3;
    }
    if (p != c) {
      for (int j = 0; j < n; ++j) {
        uint8_t t = a[c * n + j];
        a[c * n + j] = a[p * n + j];
        a[p * n + j] = t;
        t = out[c * n + j];
        out[c * n + j] = out[p * n + j];
        out[p * n + j] = t;
      }
    }
    uint8_t s = ecref_gf_inv(a[c * n + c]);
    for (int j = 0; j < n; ++j) {
      a[c * n + j] = ecref_gf_mul(a[c * n + j], s);
      out[c * n + j] = ecref_gf_mul(out[c * n + j], s);
    }
    for (int r = 0; r < n; ++r) {
      if (r == c || a[r * n + c] == 0) continue;
      uint8_t f = a[r * n + c];
      for (int j = 0; j < n; ++j) {
        a[r * n + j] ^= ecref_gf_mul(f, a[c * n + j]);
        out[r * n + j] ^= ecref_gf_mul(f, out[c * n + j]);
      }
    }
  }
  free(a);
  return 0;
}

/* Row g of the generator [I_k ; coeff] into row[k]. */
static void gen_row(const uint8_t* coeff, int k, int g, uint8_t* row) {
  if (g < k) {
    memset(row, 0, (size_t)k);
    row[g] = 1;
  } else {
    memcpy(row, coeff + (size_t)(g - k) * k, (size_t)k);
  }
}

int ecref_decode_matrix(const uint8_t* coeff, int k, int m, const int* erased,
                        int n_erased, int* survivors, uint8_t* rows) {
  if (k < 1 || m < 0 || n_erased < 0) return -1;
  if (n_erased > m) return -3;
  int n = k + m;
  char* lost = (char*)calloc((size_t)n, 1);
  for (int e = 0; e < n_erased; ++e) {
    if (erased[e] < 0 || erased[e] >= n || lost[erased[e]]) {
      free(lost);
      return -1;
    }
    lost[erased[e]] = 1;
  }
  int ns = 0;
  for (int g = 0; g < n && ns < k; ++g)
    if (!lost[g]) survivors[ns++] = g;
  free(lost);
  uint8_t* gs = (uint8_t*)malloc((size_t)k * k);
  uint8_t* inv = (uint8_t*)malloc((size_t)k * k);
  uint8_t* row = (uint8_t*)malloc((size_t)k);
  for (int s = 0; s < k; ++s) gen_row(coeff, k, survivors[s], gs + (size_t)s * k);
  int st = ecref_gf_invert(gs, inv, k);
  if (st == 0) {
    /* lost_e = G[e] . data = G[e] . inv(G_S) . survivors */
    for (int e = 0; e < n_erased; ++e) {
      gen_row(coeff, k, erased[e], row);
      for (int s = 0; s < k; ++s) {
        uint8_t acc = 0;
        for (int t = 0; t < k; ++t)
          acc ^= ecref_gf_mul(row[t], inv[(size_t)t * k + s]);
        rows[(size_t)e * k + s] = acc;
      }
    }
  }
  free(gs);
  free(inv);
  free(row);
  return st;
}

void ecref_xor_encode(const uint8_t* const* data, int k, uint8_t* parity,
                      uint64_t n) {
  for (uint64_t b = 0; b < n; ++b) {
    uint8_t acc = 0;
    for (int j = 0; j < k; ++j) acc ^= data[j][b];
    parity[b] = acc;
  }
}

static uint8_t g_mul_table[256][256];
static int g_mul_ready = 0;

static void build_mul_table(void) {
  if (g_mul_ready) return;
  for (int a = 0; a < 256; ++a)
    for (int b = 0; b < 256; ++b)
      g_mul_table[a][b] = ecref_gf_mul((uint8_t)a, (uint8_t)b);
  g_mul_ready = 1;
}

void ecref_rs_encode(const uint8_t* coeff, int k, int m,
                     const uint8_t* const* data, uint8_t* const* parity,
                     uint64_t n) {
  build_mul_table();
  for (int i = 0; i < m; ++i) {
    uint8_t* p = parity[i];
    memset(p, 0, n);
    for (int j = 0; j < k; ++j) {
      const uint8_t* t = g_mul_table[coeff[i * k + j]];
      const uint8_t* d = data[j];
      for (uint64_t b = 0; b < n; ++b) p[b] ^= t[d[b]];
    }
  }
}

void ecref_encode_batched(const uint8_t* coeff, int k, int m,
                          const uint64_t* data_ptrs, const uint32_t* data_len,
                          const uint64_t* parity_ptrs, uint32_t n_stripes,
                          uint32_t unit_bytes) {
  build_mul_table();
  for (uint32_t s = 0; s < n_stripes; ++s) {
    for (int i = 0; i < m; ++i) {
      uint8_t* p = (uint8_t*)(uintptr_t)parity_ptrs[(size_t)s * m + i];
      memset(p, 0, unit_bytes);
      for (int j = 0; j < k; ++j) {
        const uint8_t* d = (const uint8_t*)(uintptr_t)data_ptrs[(size_t)s * k + j];
        uint32_t len = d ? data_len[(size_t)s * k + j] : 0;
        if (len > unit_bytes) len = unit_bytes;
        const uint8_t* t = g_mul_table[coeff[i * k + j]];
        for (uint32_t b = 0; b < len; ++b) p[b] ^= t[d[b]];
      }
    }
  }
}

void ecref_parity_update(const uint8_t* coeff, int k, int m,
                         const uint64_t* new_ptrs, const uint64_t* old_ptrs,
                         const uint32_t* len, const uint64_t* parity_ptrs,
                         uint32_t n_stripes, uint32_t unit_bytes) {
  build_mul_table();
  for (uint32_t s = 0; s < n_stripes; ++s) {
    for (int j = 0; j < k; ++j) {
      const uint8_t* nw = (const uint8_t*)(uintptr_t)new_ptrs[(size_t)s * k + j];
      if (!nw) continue;
      const uint8_t* od = (const uint8_t*)(uintptr_t)old_ptrs[(size_t)s * k + j];
      uint32_t l = len[(size_t)s * k + j];
      if (l > unit_bytes) l = unit_bytes;
      for (int i = 0; i < m; ++i) {
        uint8_t* p = (uint8_t*)(uintptr_t)parity_ptrs[(size_t)s * m + i];
        const uint8_t* t = g_mul_table[coeff[i * k + j]];
        for (uint32_t b = 0; b < l; ++b) p[b] ^= t[(uint8_t)(nw[b] ^ od[b])];
      }
    }
  }
}
