/*
 * ec_cpu_fast.c — multithreaded SIMD CPU encoder: the timed CPU baseline.
 *
 * TEST INFRASTRUCTURE: loaded only by tests/ (as a fast checker for
 * full-size GPU outputs) and by bench.py's cpu_baseline leg.  The reference
 * ships no CPU encoder, so this is the repo's own, computing exactly the code
 * of ec_oracle.c (tests pin it to the scalar oracle byte for byte).
 *
 * Methods (picked at run time from the host's CPUID):
 *   gfni512  GF2P8AFFINEQB with the 8x8 bit matrix of "multiply by c"; works
 *            for any reduction polynomial (GF2P8MULB is fixed to 0x11B and is
 *            not used);
 *   avx512   split-nibble lookups: c*x = Tlo[x & 15] ^ Thi[x >> 4] with
 *            VPSHUFB on 64-byte vectors;
 *   avx2     the same on 32-byte vectors;
 *   scalar   product-table lookups.
 * Work is split over `nthreads` pthreads by contiguous byte ranges.
 */
#include <immintrin.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

#include "ec_oracle.h"

enum { ISA_SCALAR = 0, ISA_AVX2 = 1, ISA_AVX512 = 2, ISA_GFNI512 = 3 };
static int g_isa = -1;

static int detect_isa(void) {
  __builtin_cpu_init();
  if (__builtin_cpu_supports("avx512bw") && __builtin_cpu_supports("gfni"))
    return ISA_GFNI512;
  if (__builtin_cpu_supports("avx512bw")) return ISA_AVX512;
  if (__builtin_cpu_supports("avx2")) return ISA_AVX2;
  return ISA_SCALAR;
}

static int isa(void) {
  if (g_isa < 0) g_isa = detect_isa();
  return g_isa;
}

const char* ecfast_isa(void) {
  static const char* names[] = {"scalar", "avx2", "avx512", "gfni512"};
  return names[isa()];
}

int ecfast_force_isa(const char* name) {
  int want = -1;
  if (!strcmp(name, "scalar")) want = ISA_SCALAR;
  else if (!strcmp(name, "avx2")) want = ISA_AVX2;
  else if (!strcmp(name, "avx512")) want = ISA_AVX512;
  else if (!strcmp(name, "gfni512")) want = ISA_GFNI512;
  if (want < 0 || want > detect_isa()) return 0;
  g_isa = want;
  return 1;
}

/* ---- per-coefficient tables ------------------------------------------ */

typedef struct {
  uint8_t lo[16], hi[16]; /* c*n, c*(n<<4) for n < 16 */
  uint64_t affine;        /* GF2P8AFFINEQB matrix of multiply-by-c */
  uint8_t full[256];      /* c*x */
} coef_tab;

static void make_tab(uint8_t c, coef_tab* t) {
  for (int x = 0; x < 256; ++x) t->full[x] = ecref_gf_mul(c, (uint8_t)x);
  for (int n = 0; n < 16; ++n) {
    t->lo[n] = t->full[n];
    t->hi[n] = t->full[n << 4];
  }
  /* Output bit i = parity(row_i & x), row_i stored in byte 7-i; bit b of
   * row_i is bit i of c*2^b (column b of the multiply-by-c matrix). */
  uint64_t a = 0;
  for (int i = 0; i < 8; ++i) {
    uint8_t row = 0;
    for (int b = 0; b < 8; ++b)
      if ((t->full[1u << b] >> i) & 1u) row |= (uint8_t)(1u << b);
    a |= (uint64_t)row << (8 * (7 - i));
  }
  t->affine = a;
}

/* ---- kernels over [lo, hi) -------------------------------------------- */

typedef struct {
  const uint8_t* const* data;
  uint8_t* const* parity;
  const coef_tab* tabs; /* m*k, row-major; NULL for XOR */
  int k, m;
  uint64_t lo, hi;
  int accum; /* 1: parity ^= product (the incremental update), 0: parity = product */
} job;

static void rs_scalar(const job* J, uint64_t lo, uint64_t hi) {
  for (int i = 0; i < J->m; ++i) {
    uint8_t* p = J->parity[i];
    for (uint64_t b = lo; b < hi; ++b) {
      uint8_t acc = 0;
      for (int j = 0; j < J->k; ++j) acc ^= J->tabs[i * J->k + j].full[J->data[j][b]];
      p[b] = J->accum ? (uint8_t)(p[b] ^ acc) : acc;
    }
  }
}

__attribute__((target("avx2"))) static void rs_avx2(const job* J, uint64_t lo,
                                                    uint64_t hi) {
  const __m256i mask = _mm256_set1_epi8(0x0f);
  uint64_t b = lo;
  for (; b + 32 <= hi; b += 32) {
    __m256i acc[EC_ORACLE_MAX_M];
    for (int i = 0; i < J->m; ++i) acc[i] = _mm256_setzero_si256();
    for (int j = 0; j < J->k; ++j) {
      __m256i x = _mm256_loadu_si256((const __m256i*)(J->data[j] + b));
      __m256i xl = _mm256_and_si256(x, mask);
      __m256i xh = _mm256_and_si256(_mm256_srli_epi16(x, 4), mask);
      for (int i = 0; i < J->m; ++i) {
        const coef_tab* t = &J->tabs[i * J->k + j];
        __m256i tl = _mm256_broadcastsi128_si256(_mm_loadu_si128((const __m128i*)t->lo));
        __m256i th = _mm256_broadcastsi128_si256(_mm_loadu_si128((const __m128i*)t->hi));
        acc[i] = _mm256_xor_si256(acc[i], _mm256_xor_si256(_mm256_shuffle_epi8(tl, xl),
                                                           _mm256_shuffle_epi8(th, xh)));
      }
    }
    for (int i = 0; i < J->m; ++i) {
      if (J->accum)
        acc[i] = _mm256_xor_si256(acc[i], _mm256_loadu_si256((const __m256i*)(J->parity[i] + b)));
      _mm256_storeu_si256((__m256i*)(J->parity[i] + b), acc[i]);
    }
  }
  if (b < hi) rs_scalar(J, b, hi);
}

__attribute__((target("avx512f,avx512bw"))) static void rs_avx512(const job* J,
                                                                  uint64_t lo,
                                                                  uint64_t hi) {
  const __m512i mask = _mm512_set1_epi8(0x0f);
  uint64_t b = lo;
  for (; b + 64 <= hi; b += 64) {
    __m512i acc[EC_ORACLE_MAX_M];
    for (int i = 0; i < J->m; ++i) acc[i] = _mm512_setzero_si512();
    for (int j = 0; j < J->k; ++j) {
      __m512i x = _mm512_loadu_si512((const void*)(J->data[j] + b));
      __m512i xl = _mm512_and_si512(x, mask);
      __m512i xh = _mm512_and_si512(_mm512_srli_epi16(x, 4), mask);
      for (int i = 0; i < J->m; ++i) {
        const coef_tab* t = &J->tabs[i * J->k + j];
        __m512i tl = _mm512_broadcast_i32x4(_mm_loadu_si128((const __m128i*)t->lo));
        __m512i th = _mm512_broadcast_i32x4(_mm_loadu_si128((const __m128i*)t->hi));
        acc[i] = _mm512_ternarylogic_epi64(acc[i], _mm512_shuffle_epi8(tl, xl),
                                           _mm512_shuffle_epi8(th, xh), 0x96);
      }
    }
    for (int i = 0; i < J->m; ++i) {
      if (J->accum)
        acc[i] = _mm512_xor_si512(acc[i], _mm512_loadu_si512((const void*)(J->parity[i] + b)));
      _mm512_storeu_si512((void*)(J->parity[i] + b), acc[i]);
    }
  }
  if (b < hi) rs_scalar(J, b, hi);
}

__attribute__((target("avx512f,avx512bw,gfni"))) static void rs_gfni512(const job* J,
                                                                       uint64_t lo,
                                                                       uint64_t hi) {
  uint64_t b = lo;
  for (; b + 64 <= hi; b += 64) {
    __m512i acc[EC_ORACLE_MAX_M];
    for (int i = 0; i < J->m; ++i) acc[i] = _mm512_setzero_si512();
    for (int j = 0; j < J->k; ++j) {
      __m512i x = _mm512_loadu_si512((const void*)(J->data[j] + b));
      for (int i = 0; i < J->m; ++i) {
        __m512i a = _mm512_set1_epi64((long long)J->tabs[i * J->k + j].affine);
        acc[i] = _mm512_xor_si512(acc[i], _mm512_gf2p8affine_epi64_epi8(x, a, 0));
      }
    }
    for (int i = 0; i < J->m; ++i) {
      if (J->accum)
        acc[i] = _mm512_xor_si512(acc[i], _mm512_loadu_si512((const void*)(J->parity[i] + b)));
      _mm512_storeu_si512((void*)(J->parity[i] + b), acc[i]);
    }
  }
  if (b < hi) rs_scalar(J, b, hi);
}

static void xor_scalar(const job* J, uint64_t lo, uint64_t hi) {
  for (uint64_t b = lo; b < hi; ++b) {
    uint8_t acc = 0;
    for (int j = 0; j < J->k; ++j) acc ^= J->data[j][b];
    J->parity[0][b] = acc;
  }
}

__attribute__((target("avx2"))) static void xor_avx2(const job* J, uint64_t lo,
                                                     uint64_t hi) {
  uint64_t b = lo;
  for (; b + 32 <= hi; b += 32) {
    __m256i acc = _mm256_setzero_si256();
    for (int j = 0; j < J->k; ++j)
      acc = _mm256_xor_si256(acc, _mm256_loadu_si256((const __m256i*)(J->data[j] + b)));
    _mm256_storeu_si256((__m256i*)(J->parity[0] + b), acc);
  }
  if (b < hi) xor_scalar(J, b, hi);
}

__attribute__((target("avx512f"))) static void xor_avx512(const job* J, uint64_t lo,
                                                          uint64_t hi) {
  uint64_t b = lo;
  for (; b + 64 <= hi; b += 64) {
    __m512i acc = _mm512_setzero_si512();
    for (int j = 0; j < J->k; ++j)
      acc = _mm512_xor_si512(acc, _mm512_loadu_si512((const void*)(J->data[j] + b)));
    _mm512_storeu_si512((void*)(J->parity[0] + b), acc);
  }
  if (b < hi) xor_scalar(J, b, hi);
}

/* ---- threading -------------------------------------------------------- */

static void run_range(const job* J, uint64_t lo, uint64_t hi) {
  int s = isa();
  if (J->tabs == NULL) {
    if (s >= ISA_AVX512) xor_avx512(J, lo, hi);
    else if (s == ISA_AVX2) xor_avx2(J, lo, hi);
    else xor_scalar(J, lo, hi);
    return;
  }
  switch (s) {
    case ISA_GFNI512: rs_gfni512(J, lo, hi); break;
    case ISA_AVX512: rs_avx512(J, lo, hi); break;
    case ISA_AVX2: rs_avx2(J, lo, hi); break;
    default: rs_scalar(J, lo, hi); break;
  }
}

static void* thread_main(void* arg) {
  const job* J = (const job*)arg;
  /* Sub-blocks of 16 KiB keep the k input streams and m outputs in L1/L2. */
  const uint64_t blk = 16384;
  for (uint64_t b = J->lo; b < J->hi; b += blk) {
    uint64_t e = b + blk < J->hi ? b + blk : J->hi;
    run_range(J, b, e);
  }
  return NULL;
}

static void run_threads(job base, uint64_t n, int nthreads) {
  if (nthreads < 1) nthreads = 1;
  uint64_t per = (n + (uint64_t)nthreads - 1) / (uint64_t)nthreads;
  per = (per + 63) & ~(uint64_t)63;
  if (per == 0) per = 64;
  pthread_t* th = (pthread_t*)calloc((size_t)nthreads, sizeof(pthread_t));
  char* created = (char*)calloc((size_t)nthreads, 1);
  job* jobs = (job*)calloc((size_t)nthreads, sizeof(job));
  for (int t = 0; t < nthreads; ++t) {
    uint64_t lo = (uint64_t)t * per;
    if (lo >= n) break;
    jobs[t] = base;
    jobs[t].lo = lo;
    jobs[t].hi = lo + per < n ? lo + per : n;
    /* The calling thread takes the last range itself. */
    if (t == nthreads - 1 || pthread_create(&th[t], NULL, thread_main, &jobs[t]) != 0)
      thread_main(&jobs[t]);
    else
      created[t] = 1;
  }
  for (int t = 0; t < nthreads; ++t)
    if (created[t]) pthread_join(th[t], NULL);
  free(th);
  free(created);
  free(jobs);
}

void ecfast_xor_encode(const uint8_t* const* data, int k, uint8_t* parity,
                       uint64_t n, int nthreads) {
  uint8_t* const par[1] = {parity};
  job base = {data, par, NULL, k, 1, 0, 0, 0};
  run_threads(base, n, nthreads);
}

void ecfast_rs_encode(const uint8_t* coeff, int k, int m,
                      const uint8_t* const* data, uint8_t* const* parity,
                      uint64_t n, int nthreads) {
  if (m > EC_ORACLE_MAX_M) return;
  /* aligned_alloc wants the size to be a multiple of the alignment */
  const size_t bytes = (sizeof(coef_tab) * (size_t)(k * m) + 63) & ~(size_t)63;
  coef_tab* tabs = (coef_tab*)aligned_alloc(64, bytes);
  for (int i = 0; i < m * k; ++i) make_tab(coeff[i], &tabs[i]);
  job base = {data, parity, tabs, k, m, 0, 0, 0};
  run_threads(base, n, nthreads);
  free(tabs);
}

/* ---- batched stripes (configs 4 and 5) -------------------------------- */

typedef struct {
  const uint64_t* dptr; /* [S][k], 0 = absent (update: the new bytes, 0 = unchanged) */
  const uint32_t* dlen; /* [S][k] valid bytes */
  const uint64_t* pptr; /* [S][m] */
  const coef_tab* tabs;
  int k, m;
  uint32_t unit_bytes;
  uint32_t s_lo, s_hi;  /* stripes of this thread */
  const uint64_t* optr; /* update: [S][k] the old bytes; NULL for the encode */
} bjob;

/* d[b] = a[b] ^ b_[b] for b < n (any alignment). */
__attribute__((target("avx512f"))) static void xor_bytes_avx512(uint8_t* d, const uint8_t* a,
                                                                const uint8_t* b_, uint32_t n) {
  uint32_t b = 0;
  for (; b + 64 <= n; b += 64)
    _mm512_storeu_si512((void*)(d + b), _mm512_xor_si512(_mm512_loadu_si512((const void*)(a + b)),
                                                         _mm512_loadu_si512((const void*)(b_ + b))));
  for (; b < n; ++b) d[b] = a[b] ^ b_[b];
}

static void xor_bytes(uint8_t* d, const uint8_t* a, const uint8_t* b_, uint32_t n) {
  if (isa() >= ISA_AVX512) {
    xor_bytes_avx512(d, a, b_, n);
    return;
  }
  for (uint32_t b = 0; b < n; ++b) d[b] = a[b] ^ b_[b];
}

/* Stripes [s_lo, s_hi): units with all unit_bytes valid are read in place;
 * a short or absent unit is copied, zero-padded, into this thread's
 * k x unit_bytes scratch (the code treats bytes past a unit's length as
 * zeros, as ecref_encode_batched does). */
static void* bthread_main(void* arg) {
  const bjob* B = (const bjob*)arg;
  const uint32_t U = B->unit_bytes;
  uint8_t* scratch = NULL;
  const uint8_t* data[64];
  uint8_t* par[EC_ORACLE_MAX_M];
  for (uint32_t s = B->s_lo; s < B->s_hi; ++s) {
    for (int j = 0; j < B->k; ++j) {
      const uint8_t* p = (const uint8_t*)(uintptr_t)B->dptr[(uint64_t)s * B->k + j];
      uint32_t len = p ? B->dlen[(uint64_t)s * B->k + j] : 0;
      if (len > U) len = U;
      if (len == U) {
        data[j] = p;
        continue;
      }
      if (!scratch && !(scratch = (uint8_t*)malloc((size_t)B->k * U))) return (void*)1;
      uint8_t* pad = scratch + (size_t)j * U;
      if (len) memcpy(pad, p, len);
      memset(pad + len, 0, U - len);
      data[j] = pad;
    }
    for (int i = 0; i < B->m; ++i)
      par[i] = (uint8_t*)(uintptr_t)B->pptr[(uint64_t)s * B->m + i];
    job J = {data, par, B->tabs, B->k, B->m, 0, U, 0};
    thread_main(&J);
  }
  free(scratch);
  return NULL;
}

/* Stripes of the incremental update: for each changed unit j of stripe s
 * (new_ptrs[s][j] != 0) delta_j = new_j ^ old_j over its valid bytes, then
 * parity_i ^= XOR_j C[i][j] * delta_j over the longest changed unit's bytes,
 * through the encode kernels in accumulate mode with the coefficient columns
 * of the changed units only (bytes past a unit's length have a zero delta;
 * parity bytes past the longest changed unit are unchanged). */
static void* uthread_main(void* arg) {
  const bjob* B = (const bjob*)arg;
  const uint32_t U = B->unit_bytes;
  uint8_t* scratch = NULL;
  const uint8_t* delta[64];
  uint8_t* par[EC_ORACLE_MAX_M];
  coef_tab* sub = NULL;
  for (uint32_t s = B->s_lo; s < B->s_hi; ++s) {
    int nc = 0;
    uint32_t lmax = 0;
    for (int j = 0; j < B->k; ++j) {
      const uint8_t* nw = (const uint8_t*)(uintptr_t)B->dptr[(uint64_t)s * B->k + j];
      if (!nw) continue;
      const uint8_t* od = (const uint8_t*)(uintptr_t)B->optr[(uint64_t)s * B->k + j];
      uint32_t len = B->dlen[(uint64_t)s * B->k + j];
      if (len > U) len = U;
      if (!scratch) {
        scratch = (uint8_t*)malloc((size_t)B->k * U);
        sub = (coef_tab*)malloc(sizeof(coef_tab) * (size_t)(B->k * B->m));
        if (!scratch || !sub) {
          free(scratch);
          free(sub);
          return (void*)1;
        }
      }
      uint8_t* d = scratch + (size_t)nc * U;
      xor_bytes(d, nw, od, len);
      memset(d + len, 0, U - len);
      delta[nc] = d;
      for (int i = 0; i < B->m; ++i) sub[i * B->k + nc] = B->tabs[i * B->k + j];
      lmax = len > lmax ? len : lmax;
      ++nc;
    }
    if (nc == 0 || lmax == 0) continue;
    /* sub holds the changed columns at row stride k; compact it to stride nc
     * (the layout the kernels read) */
    for (int i = 1; i < B->m; ++i)
      memmove(&sub[i * nc], &sub[i * B->k], sizeof(coef_tab) * (size_t)nc);
    for (int i = 0; i < B->m; ++i)
      par[i] = (uint8_t*)(uintptr_t)B->pptr[(uint64_t)s * B->m + i];
    job J = {delta, par, sub, nc, B->m, 0, lmax, 1};
    thread_main(&J);
  }
  free(scratch);
  free(sub);
  return NULL;
}

/* Whole stripes per thread: n_stripes split into nthreads contiguous shares,
 * the calling thread taking the last one.  0, or -1 when a thread failed. */
static int run_stripe_threads(bjob base, uint32_t n_stripes, int nthreads,
                              void* (*fn)(void*)) {
  if (nthreads < 1) nthreads = 1;
  if ((uint32_t)nthreads > n_stripes) nthreads = n_stripes ? (int)n_stripes : 1;
  pthread_t* th = (pthread_t*)calloc((size_t)nthreads, sizeof(pthread_t));
  char* created = (char*)calloc((size_t)nthreads, 1);
  bjob* jobs = (bjob*)calloc((size_t)nthreads, sizeof(bjob));
  int status = (th && created && jobs) ? 0 : -1;
  const uint32_t per = n_stripes / (uint32_t)nthreads, extra = n_stripes % (uint32_t)nthreads;
  uint32_t s0 = 0;
  for (int t = 0; status == 0 && t < nthreads; ++t) {
    const uint32_t cnt = per + ((uint32_t)t < extra ? 1u : 0u);
    jobs[t] = base;
    jobs[t].s_lo = s0;
    jobs[t].s_hi = s0 + cnt;
    s0 += cnt;
    if (t == nthreads - 1 || pthread_create(&th[t], NULL, fn, &jobs[t]) != 0) {
      if (fn(&jobs[t]) != NULL) status = -1;
    } else {
      created[t] = 1;
    }
  }
  for (int t = 0; t < nthreads; ++t) {
    void* r = NULL;
    if (created[t] && pthread_join(th[t], &r) == 0 && r != NULL) status = -1;
  }
  free(th);
  free(created);
  free(jobs);
  return status;
}

static coef_tab* make_tabs(const uint8_t* coeff, int k, int m) {
  const size_t bytes = (sizeof(coef_tab) * (size_t)(k * m) + 63) & ~(size_t)63;
  coef_tab* tabs = (coef_tab*)aligned_alloc(64, bytes);
  if (tabs)
    for (int i = 0; i < m * k; ++i) make_tab(coeff[i], &tabs[i]);
  return tabs;
}

int ecfast_encode_batched(const uint8_t* coeff, int k, int m, const uint64_t* data_ptrs,
                          const uint32_t* data_len, const uint64_t* parity_ptrs,
                          uint32_t n_stripes, uint32_t unit_bytes, int nthreads) {
  if (k < 1 || k > 64 || m < 1 || m > EC_ORACLE_MAX_M) return -1;
  coef_tab* tabs = make_tabs(coeff, k, m);
  if (!tabs) return -1;
  bjob b = {data_ptrs, data_len, parity_ptrs, tabs, k, m, unit_bytes, 0, 0, NULL};
  const int status = run_stripe_threads(b, n_stripes, nthreads, bthread_main);
  free(tabs);
  return status;
}

int ecfast_parity_update(const uint8_t* coeff, int k, int m, const uint64_t* new_ptrs,
                         const uint64_t* old_ptrs, const uint32_t* len,
                         const uint64_t* parity_ptrs, uint32_t n_stripes, uint32_t unit_bytes,
                         int nthreads) {
  if (k < 1 || k > 64 || m < 1 || m > EC_ORACLE_MAX_M || !old_ptrs) return -1;
  coef_tab* tabs = make_tabs(coeff, k, m);
  if (!tabs) return -1;
  bjob b = {new_ptrs, len, parity_ptrs, tabs, k, m, unit_bytes, 0, 0, old_ptrs};
  const int status = run_stripe_threads(b, n_stripes, nthreads, uthread_main);
  free(tabs);
  return status;
}
