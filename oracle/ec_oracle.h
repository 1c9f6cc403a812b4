/*
 * ec_oracle.h — CPU oracle for the erasure-coding hot path.
 *
 * TEST INFRASTRUCTURE.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this code, and only as the checker
 * or the timed CPU baseline.  The product (megatron-lm_amd/) never calls it.
 *
 * The reference (duihuhu/Megatron-LM) contains no erasure coder in any
 * language, so there is no reference file:line to follow for the arithmetic.
 * This is a restatement from the mathematics of the code the engine
 * computes:
 *   field      GF(2^8), reduction polynomial 0x11D, generator 0x02
 *   generator  G = [I_k ; C], C[i][j] = inv((k+i) ^ j)   (Cauchy matrix)
 *   encode     parity_i[b] = XOR_j C[i][j] * data_j[b]
 *   XOR        parity[b]   = XOR_j data_j[b]
 *   decode     invert the k x k rows of G of the first k surviving shards
 * and of the reference path's data shapes it serves: the ragged tensor list
 * of megatron/core/dist_checkpointing/tensor_aware_state_dict.py:179-184,
 * chunked in order into fixed-size units.
 *
 * What pins it (tests/test_oracle.py): brute force of every product against
 * carry-less multiply mod 0x11D, the field axioms, the published
 * ISO/IEC 18004 (QR code) Reed-Solomon example over the same field, the MDS
 * property over every erasure pattern, unit-vector responses, linearity, an
 * independent pure-Python restatement (oracle/pyref.py) and the committed
 * golden vectors under tests/golden/.
 */
#ifndef EC_ORACLE_H
#define EC_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* scalar oracle (ec_oracle.c) */
uint8_t ecref_gf_mul(uint8_t a, uint8_t b);
uint8_t ecref_gf_inv(uint8_t a);
int ecref_cauchy(int k, int m, uint8_t* out);
int ecref_gf_invert(const uint8_t* in, uint8_t* out, int n);
int ecref_decode_matrix(const uint8_t* coeff, int k, int m, const int* erased,
                        int n_erased, int* survivors, uint8_t* rows);
void ecref_xor_encode(const uint8_t* const* data, int k, uint8_t* parity,
                      uint64_t n);
void ecref_rs_encode(const uint8_t* coeff, int k, int m,
                     const uint8_t* const* data, uint8_t* const* parity,
                     uint64_t n);
void ecref_encode_batched(const uint8_t* coeff, int k, int m,
                          const uint64_t* data_ptrs, const uint32_t* data_len,
                          const uint64_t* parity_ptrs, uint32_t n_stripes,
                          uint32_t unit_bytes);
void ecref_parity_update(const uint8_t* coeff, int k, int m,
                         const uint64_t* new_ptrs, const uint64_t* old_ptrs,
                         const uint32_t* len, const uint64_t* parity_ptrs,
                         uint32_t n_stripes, uint32_t unit_bytes);

/* multithreaded SIMD CPU encoder (ec_cpu_fast.c), the timed CPU baseline;
 * m <= EC_ORACLE_MAX_M */
#define EC_ORACLE_MAX_M 16
const char* ecfast_isa(void);
void ecfast_xor_encode(const uint8_t* const* data, int k, uint8_t* parity,
                       uint64_t n, int nthreads);
void ecfast_rs_encode(const uint8_t* coeff, int k, int m,
                      const uint8_t* const* data, uint8_t* const* parity,
                      uint64_t n, int nthreads);
/* ecref_encode_batched's stripes on nthreads threads (whole stripes per
 * thread); 0, or -1 for bad arguments or out of memory */
int ecfast_encode_batched(const uint8_t* coeff, int k, int m, const uint64_t* data_ptrs,
                          const uint32_t* data_len, const uint64_t* parity_ptrs,
                          uint32_t n_stripes, uint32_t unit_bytes, int nthreads);
/* ecref_parity_update's stripes on nthreads threads (whole stripes per
 * thread); 0, or -1 for bad arguments or out of memory */
int ecfast_parity_update(const uint8_t* coeff, int k, int m, const uint64_t* new_ptrs,
                         const uint64_t* old_ptrs, const uint32_t* len,
                         const uint64_t* parity_ptrs, uint32_t n_stripes, uint32_t unit_bytes,
                         int nthreads);
/* force an ISA ("gfni512", "avx512", "avx2", "scalar"); 0 if unsupported */
int ecfast_force_isa(const char* name);

#ifdef __cplusplus
}
#endif

#endif
