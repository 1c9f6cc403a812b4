/* Host-side driver for the sanitizer test: exercises the C oracle, the SIMD
 * CPU encoder and the engine's host GF(2^8) code (ec_gf_*, ec_cauchy_matrix,
 * ec_gf_invert, ec_decode_matrix) on small and edge-case inputs, under
 * AddressSanitizer and UndefinedBehaviorSanitizer.  Exit 0 = all checks hold. */
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "ec_mi355.h"
#include "ec_oracle.h"

#define FAIL(...) do { fprintf(stderr, __VA_ARGS__); fputc('\n', stderr); return 1; } while (0)

static uint32_t s = 12345u;
static uint8_t r8(void) { s = s * 1103515245u + 12345u; return (uint8_t)(s >> 16); }

int main(void) {
  /* field: product code vs oracle, all pairs */
  for (int a = 0; a < 256; ++a)
    for (int b = 0; b < 256; ++b)
      if (ec_gf_mul((uint8_t)a, (uint8_t)b) != ecref_gf_mul((uint8_t)a, (uint8_t)b)) FAIL("mul %d %d", a, b);
  for (int a = 0; a < 256; ++a)
    if (ec_gf_inv((uint8_t)a) != ecref_gf_inv((uint8_t)a)) FAIL("inv %d", a);

  const int shapes[][2] = {{1, 1}, {4, 1}, {6, 3}, {8, 2}, {12, 4}, {16, 4}, {32, 16}, {200, 56}};
  for (size_t t = 0; t < sizeof shapes / sizeof shapes[0]; ++t) {
    int k = shapes[t][0], m = shapes[t][1];
    uint8_t* c1 = malloc((size_t)k * m);
    uint8_t* c2 = malloc((size_t)k * m);
    if (ec_cauchy_matrix(k, m, c1) != EC_OK || ecref_cauchy(k, m, c2) != 0) FAIL("cauchy %d %d", k, m);
    if (memcmp(c1, c2, (size_t)k * m)) FAIL("cauchy differs %d %d", k, m);
    /* decode plans for a few erasure patterns, product vs oracle */
    if (k + m <= 64) {
      int er[16], sv1[64], sv2[64];
      uint8_t* r1 = malloc((size_t)m * k);
      uint8_t* r2 = malloc((size_t)m * k);
      for (int rep = 0; rep < 20; ++rep) {
        int e = 1 + rep % m, n = 0;
        while (n < e) {
          int g = r8() % (k + m), dup = 0;
          for (int q = 0; q < n; ++q) dup |= er[q] == g;
          if (!dup) er[n++] = g;
        }
        int a = ec_decode_matrix(c1, k, m, er, e, sv1, r1);
        int b = ecref_decode_matrix(c2, k, m, er, e, sv2, r2);
        if (a != EC_OK || b != 0) FAIL("decode plan %d %d", a, b);
        if (memcmp(sv1, sv2, sizeof(int) * k) || memcmp(r1, r2, (size_t)e * k)) FAIL("plan differs");
      }
      /* too many erasures, duplicate and out-of-range indices */
      int bad[17];
      for (int q = 0; q <= m && q < 17; ++q) bad[q] = q;
      if (ec_decode_matrix(c1, k, m, bad, m + 1, sv1, r1) != EC_ESINGULAR) FAIL("m+1 erasures");
      int dup2[2] = {0, 0};
      if (m >= 2 && ec_decode_matrix(c1, k, m, dup2, 2, sv1, r1) != EC_EINVAL) FAIL("duplicate");
      int oor[1] = {k + m};
      if (ec_decode_matrix(c1, k, m, oor, 1, sv1, r1) != EC_EINVAL) FAIL("out of range");
      free(r1);
      free(r2);
    }
    free(c1);
    free(c2);
  }
  /* invert: random matrices, singular ones */
  for (int n = 1; n <= 12; ++n) {
    uint8_t *A = malloc((size_t)n * n), *B = malloc((size_t)n * n), *C = malloc((size_t)n * n);
    for (int i = 0; i < n * n; ++i) A[i] = r8();
    int a = ec_gf_invert(A, B, n), b = ecref_gf_invert(A, C, n);
    if ((a == EC_OK) != (b == 0)) FAIL("invert status %d", n);
    if (a == EC_OK && memcmp(B, C, (size_t)n * n)) FAIL("invert differs %d", n);
    memset(A, 0, (size_t)n * n);
    if (ec_gf_invert(A, B, n) != EC_ESINGULAR) FAIL("zero matrix");
    free(A); free(B); free(C);
  }
  if (ec_cauchy_matrix(0, 1, NULL) != EC_EINVAL || ec_cauchy_matrix(200, 57, (uint8_t*)&s) != EC_ERANGE)
    FAIL("cauchy errors");

  /* encoders: scalar oracle vs SIMD baseline, odd sizes, threads */
  const uint64_t sizes[] = {1, 15, 63, 64, 65, 1000, 4096 + 7};
  for (size_t z = 0; z < sizeof sizes / sizeof sizes[0]; ++z) {
    uint64_t n = sizes[z];
    int k = 6, m = 3;
    uint8_t coeff[18];
    ec_cauchy_matrix(k, m, coeff);
    uint8_t* d[6];
    uint8_t* p1[3];
    uint8_t* p2[3];
    for (int j = 0; j < k; ++j) { d[j] = malloc(n); for (uint64_t b = 0; b < n; ++b) d[j][b] = r8(); }
    for (int i = 0; i < m; ++i) { p1[i] = malloc(n); p2[i] = malloc(n); }
    ecref_rs_encode(coeff, k, m, (const uint8_t* const*)d, p1, n);
    ecfast_rs_encode(coeff, k, m, (const uint8_t* const*)d, p2, n, 3);
    for (int i = 0; i < m; ++i) if (memcmp(p1[i], p2[i], n)) FAIL("fast rs %llu", (unsigned long long)n);
    ecref_xor_encode((const uint8_t* const*)d, k, p1[0], n);
    ecfast_xor_encode((const uint8_t* const*)d, k, p2[0], n, 2);
    if (memcmp(p1[0], p2[0], n)) FAIL("fast xor");
    for (int j = 0; j < k; ++j) free(d[j]);
    for (int i = 0; i < m; ++i) { free(p1[i]); free(p2[i]); }
  }
  /* batched + update on a ragged grid with an absent slot */
  {
    enum { K = 3, M = 2, U = 48, S = 2 };
    uint8_t coeff[M * K];
    ec_cauchy_matrix(K, M, coeff);
    uint8_t* u[S * K];
    uint64_t dp[S * K], np[S * K], op[S * K], pp[S * M];
    uint32_t ln[S * K];
    uint8_t par[S * M * U], par2[S * M * U];
    for (int q = 0; q < S * K; ++q) {
      ln[q] = q == S * K - 1 ? 0 : (uint32_t)(1 + r8() % U);
      u[q] = q == S * K - 1 ? NULL : malloc(ln[q]);
      for (uint32_t b = 0; b < ln[q]; ++b) u[q][b] = r8();
      dp[q] = (uint64_t)(uintptr_t)u[q];
      np[q] = 0;
      op[q] = 0;
    }
    for (int q = 0; q < S * M; ++q) pp[q] = (uint64_t)(uintptr_t)(par + (size_t)q * U);
    ecref_encode_batched(coeff, K, M, dp, ln, pp, S, U);
    uint8_t old[U], par0[S * M * U];
    memcpy(par0, par, sizeof par);
    memcpy(old, u[1], ln[1]);
    for (uint32_t b = 0; b < ln[1]; ++b) u[1][b] ^= r8();
    np[1] = dp[1];
    op[1] = (uint64_t)(uintptr_t)old;
    ecref_parity_update(coeff, K, M, np, op, ln, pp, S, U);
    memcpy(par2, par, sizeof par);
    ecref_encode_batched(coeff, K, M, dp, ln, pp, S, U);
    if (memcmp(par, par2, sizeof par)) FAIL("update != re-encode");
    /* the SIMD batched encoder on the same grid (short units read only up
     * to their length, the absent slot as zeros), 1 and 4 threads */
    for (int th = 1; th <= 4; th += 3) {
      uint8_t par3[S * M * U];
      uint64_t pp3[S * M];
      memset(par3, 0xEE, sizeof par3);
      for (int q = 0; q < S * M; ++q) pp3[q] = (uint64_t)(uintptr_t)(par3 + (size_t)q * U);
      if (ecfast_encode_batched(coeff, K, M, dp, ln, pp3, S, U, th) != 0) FAIL("fast batched");
      if (memcmp(par3, par, sizeof par)) FAIL("fast batched differs (%d threads)", th);
      /* the SIMD update from the parity before the change */
      memcpy(par3, par0, sizeof par3);
      if (ecfast_parity_update(coeff, K, M, np, op, ln, pp3, S, U, th) != 0) FAIL("fast update");
      if (memcmp(par3, par, sizeof par)) FAIL("fast update differs (%d threads)", th);
    }
    for (int q = 0; q < S * K; ++q) free(u[q]);
  }
  printf("sanitize driver ok\n");
  return 0;
}
