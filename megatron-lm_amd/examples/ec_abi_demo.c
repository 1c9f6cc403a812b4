/*
 * ec_abi_demo.c — a plain-C caller of the engine's C ABI, as a non-Python
 * binding (cgo, JNI, N-API) would use it: device buffers from hipMalloc, an
 * explicit stream, status codes.  Encodes RS(6,3) over 6 shards, loses 3
 * seeded shards, reconstructs them and checks them byte for byte; does the
 * same for XOR parity; then codes the shards as one stripe into a snapshot
 * block (ec_encode_batched_copy) and stages the block to host memory
 * (ec_stage_to_host, then ec_stage_stripes_to_host on a copy engine), as a
 * background checkpoint save does, checking every row.  Prints
 * "ec_abi_demo ok" and exits 0 on success.
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
  /* a checkpoint snapshot: the 6 shards as the units of one stripe, coded
   * into a (6 + 3) x unit block in one pass, then staged to host memory on an
   * ordinary stream through a pinned buffer */
  {
    const uint64_t unit = (n + 15) & ~(uint64_t)15;
    if (unit > (1ull << 31)) return 6;
    uint8_t* block;
    CHECK_HIP(hipMalloc((void**)&block, (K + M) * unit));
    uint64_t h_desc[K + M + K];
    uint32_t h_len[K];
    for (int j = 0; j < K; ++j) {
      h_desc[j] = (uint64_t)(uintptr_t)dev[j];                    /* units */
      h_desc[K + M + j] = (uint64_t)(uintptr_t)(block + j * unit);  /* copies */
      h_len[j] = (uint32_t)n;
    }
    for (int i = 0; i < M; ++i) h_desc[K + i] = (uint64_t)(uintptr_t)(block + (K + i) * unit);
    uint64_t* d_desc;
    uint32_t* d_len;
    CHECK_HIP(hipMalloc((void**)&d_desc, sizeof h_desc));
    CHECK_HIP(hipMalloc((void**)&d_len, sizeof h_len));
    CHECK_HIP(hipMemcpy(d_desc, h_desc, sizeof h_desc, hipMemcpyHostToDevice));
    CHECK_HIP(hipMemcpy(d_len, h_len, sizeof h_len, hipMemcpyHostToDevice));
    CHECK_EC(ec_encode_batched_copy(coeff, K, M, d_desc, d_len, d_desc + K, d_desc + K + M, 1,
                                    (uint32_t)unit, st));
    CHECK_HIP(hipStreamSynchronize((hipStream_t)st));
    hipStream_t xfer;
    CHECK_HIP(hipStreamCreate(&xfer));
    const uint64_t pinned_bytes = 1u << 24; /* smaller than the block for large shards */
    uint8_t* pinned;
    CHECK_HIP(hipHostMalloc((void**)&pinned, pinned_bytes, hipHostMallocDefault));
    uint8_t* slices = (uint8_t*)malloc((K + M) * unit);
    CHECK_EC(ec_stage_to_host(block, unit, slices, unit, K + M, unit, pinned, pinned_bytes, 4,
                              (ec_stream_t)xfer));
    for (int g = 0; g < K + M; ++g) {
      const uint8_t* row = slices + g * unit;
      if (memcmp(row, host[g], n) != 0) {
        fprintf(stderr, "snapshot row %d differs\n", g);
        return 1;
      }
      for (uint64_t b = n; b < unit; ++b)
        if (row[b] != 0) {
          fprintf(stderr, "snapshot row %d not zero-padded\n", g);
          return 1;
        }
    }
    /* the same block, stripe-major (one stripe of K + M units), to one host
     * row per position: copies on an SDMA engine (runtime-allocated block
     * and pinned buffer), which the call's timings report */
    memset(slices, 0x5a, (K + M) * unit);
    uint8_t* rows_p[K + M];
    for (int g = 0; g < K + M; ++g) rows_p[g] = slices + g * unit;
    CHECK_EC(ec_stage_stripes_to_host(block, 1, K + M, unit, rows_p, pinned, pinned_bytes, 4,
                                      (ec_stream_t)xfer));
    ec_stage_stats stats;
    CHECK_EC(ec_stage_last_stats(&stats));
    if (stats.copy_engine != 1) {
      fprintf(stderr, "stripe staging did not run on a copy engine\n");
      return 1;
    }
    for (int g = 0; g < K + M; ++g)
      if (memcmp(slices + g * unit, host[g], n) != 0) {
        fprintf(stderr, "stripe-staged row %d differs\n", g);
        return 1;
      }
    free(slices);
    CHECK_HIP(hipHostFree(pinned));
    CHECK_HIP(hipStreamDestroy(xfer));
    CHECK_HIP(hipFree(d_desc));
    CHECK_HIP(hipFree(d_len));
    CHECK_HIP(hipFree(block));
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
