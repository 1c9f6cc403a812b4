/*
 * ec_abi_demo.c — a plain-C caller of the engine's C ABI, as a non-Python
 * binding (cgo, JNI, N-API) would use it: device buffers from hipMalloc, an
 * explicit stream, status codes.  Encodes RS(6,3) over 6 shards, loses 3
 * seeded shards, reconstructs them and checks them byte for byte; does the
 * same for XOR parity.  Prints "ec_abi_demo ok" and exits 0 on success.
 *
 *   ec_abi_demo [shard_bytes]
 */
#include <hip/hip_runtime_api.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "ec_mi355.h"

#define CHECK_HIP(x)                                                       \
  do {                                                                     \
    hipError_t e_ = (x);                                                   \
    if (e_ != hipSuccess) {                                                \
      fprintf(stderr, "%s:%d %s: %s\n", __FILE__, __LINE__, #x,            \
              hipGetErrorString(e_));                                      \
      return 2;                                                            \
    }                                                                      \
  } while (0)
#define CHECK_EC(x)                                                        \
  do {                                                                     \
    int s_ = (x);                                                          \
    if (s_ != EC_OK) {                                                     \
      fprintf(stderr, "%s:%d %s: %s\n", __FILE__, __LINE__, #x,            \
              ec_strerror(s_));                                            \
      return 3;                                                            \
    }                                                                      \
  } while (0)

static uint64_t rng_state = 0x9E3779B97F4A7C15ull;
static uint8_t rnd8(void) {
  rng_state ^= rng_state << 13;
  rng_state ^= rng_state >> 7;
  rng_state ^= rng_state << 17;
  return (uint8_t)rng_state;
}

int main(int argc, char** argv) {
  enum { K = 6, M = 3 };
  const uint64_t n = argc > 1 ? strtoull(argv[1], NULL, 0) : (1u << 20) + 3;
  if (ec_abi_version() != EC_ABI_VERSION) return 4;
  /* a stream with its own hardware queue, as checkpoint work beside training uses */
  ec_stream_t st;
  CHECK_EC(ec_stream_create(0, 0, &st));

  uint8_t* host[K + M];
  uint8_t* dev[K + M];
  for (int g = 0; g < K + M; ++g) {
    host[g] = (uint8_t*)malloc(n);
    CHECK_HIP(hipMalloc((void**)&dev[g], n));
  }
  for (int j = 0; j < K; ++j) {
    for (uint64_t b = 0; b < n; ++b) host[j][b] = rnd8();
    CHECK_HIP(hipMemcpy(dev[j], host[j], n, hipMemcpyHostToDevice));
  }

  /* encode */
  uint8_t coeff[M * K];
  CHECK_EC(ec_cauchy_matrix(K, M, coeff));
  CHECK_EC(ec_rs_encode(coeff, K, M, (const uint8_t* const*)dev, dev + K, n, st));
  CHECK_HIP(hipStreamSynchronize((hipStream_t)st));
  for (int i = 0; i < M; ++i) CHECK_HIP(hipMemcpy(host[K + i], dev[K + i], n, hipMemcpyDeviceToHost));

  /* lose shards 1, 4 and 7 (two data, one parity), rebuild them */
  const int lost[3] = {1, 4, 7};
  int surv[K];
  uint8_t rows[3 * K];
  CHECK_EC(ec_decode_matrix(coeff, K, M, lost, 3, surv, rows));
  const uint8_t* sv[K];
  for (int s = 0; s < K; ++s) sv[s] = dev[surv[s]];
  uint8_t* out[3];
  for (int r = 0; r < 3; ++r) CHECK_HIP(hipMalloc((void**)&out[r], n));
  CHECK_EC(ec_rs_decode(rows, K, 3, sv, out, n, st));
  CHECK_HIP(hipStreamSynchronize((hipStream_t)st));
  uint8_t* chk = (uint8_t*)malloc(n);
  for (int r = 0; r < 3; ++r) {
    CHECK_HIP(hipMemcpy(chk, out[r], n, hipMemcpyDeviceToHost));
    if (memcmp(chk, host[lost[r]], n) != 0) {
      fprintf(stderr, "reconstructed shard %d differs\n", lost[r]);
      return 1;
    }
  }

  /* XOR parity of the first 4 shards, checked against a host XOR */
  CHECK_EC(ec_xor_encode((const uint8_t* const*)dev, 4, out[0], n, st));
  CHECK_HIP(hipStreamSynchronize((hipStream_t)st));
  CHECK_HIP(hipMemcpy(chk, out[0], n, hipMemcpyDeviceToHost));
  for (uint64_t b = 0; b < n; ++b) {
    if (chk[b] != (uint8_t)(host[0][b] ^ host[1][b] ^ host[2][b] ^ host[3][b])) {
      fprintf(stderr, "XOR parity differs at byte %llu\n", (unsigned long long)b);
      return 1;
    }
  }
  /* too many erasures is an error, not a crash */
  const int four[4] = {0, 1, 2, 3};
  if (ec_decode_matrix(coeff, K, M, four, 4, surv, rows) != EC_ESINGULAR) return 5;

  for (int g = 0; g < K + M; ++g) {
    CHECK_HIP(hipFree(dev[g]));
    free(host[g]);
  }
  for (int r = 0; r < 3; ++r) CHECK_HIP(hipFree(out[r]));
  free(chk);
  CHECK_EC(ec_stream_destroy(st));
  printf("ec_abi_demo ok (%llu-byte shards)\n", (unsigned long long)n);
  return 0;
}
