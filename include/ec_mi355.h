/*
 * ec_mi355.h — C ABI of the MI355X (gfx950) erasure-coding engine.
 *
 * The engine computes XOR parity and systematic Reed-Solomon codes over
 * GF(2^8) (reduction polynomial x^8+x^4+x^3+x^2+1 = 0x11D, generator 0x02)
 * on device-resident checkpoint shards, and reconstructs lost shards.
 *
 * Code conventions (fixed; every entry point follows them):
 *   - generator matrix G = [ I_k ; C ] with the m x k Cauchy block
 *       C[i][j] = inv((k + i) XOR j),   i in [0, m), j in [0, k);
 *   - parity_i[b] = XOR_j C[i][j] * data_j[b] for every byte offset b;
 *   - XOR parity is plain XOR of the data shards (not the m = 1 Cauchy row);
 *   - matrices are row-major uint8 arrays in host memory.
 *
 * Where it plugs into the reference.  The reference (a Megatron-Core
 * 0.14.0rc6 fork) has no erasure coder.  Its local ("non-persistent")
 * checkpoint path hands the list of shard tensors of a
 * MCoreTensorAwareStateDict to an external LocalCheckpointManager, whose
 * redundancy step is a replication strategy injected at
 *   megatron/training/training.py:825-835   (repl_strategy=...)
 * and invoked from
 *   megatron/training/checkpointing.py:538-541  (manager.save: encode here)
 *   megatron/training/checkpointing.py:891-894  (manager.load: decode here)
 * on the tensor list of
 *   megatron/core/dist_checkpointing/tensor_aware_state_dict.py:179-243.
 * Each entry point below names the slot of that path it serves.
 *
 * ABI conventions:
 *   - every function returns EC_OK (0) or a negative EC_E* status; no C++
 *     exception crosses this boundary;
 *   - "d_" arguments are device pointers (HBM); other pointers are host;
 *   - the caller owns every buffer; the library allocates no device memory;
 *   - device work is enqueued on `stream` (a hipStream_t; NULL = the legacy
 *     default stream) and is asynchronous with respect to the host;
 *   - calls on different streams from different host threads are safe: the
 *     library keeps no mutable global state (only each thread's timings of
 *     its last staging call, ec_stage_last_stats).
 */
#ifndef EC_MI355_H
#define EC_MI355_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* 2: ec_stage_stripes_to_host added; the batched kernels read every
 * descriptor entry of a stripe, also the length of an absent unit.
 * 3: ec_stage_stripes_to_host and ec_stage_to_host copy on an SDMA engine
 * (see there); ec_stage_stats.copy_engine added. */
#define EC_ABI_VERSION 3

/* Status codes. */
#define EC_OK 0
#define EC_EINVAL (-1)    /* bad argument: k, m, size, null pointer      */
#define EC_EALIGN (-2)    /* pointer not 16-byte aligned where required   */
#define EC_ESINGULAR (-3) /* matrix not invertible / too many erasures    */
#define EC_EHIP (-4)      /* a HIP runtime call failed                    */
#define EC_ERANGE (-5)    /* k, m or a length beyond the supported limits */

/* Limits.  k + m <= 256 is what a Cauchy code over GF(2^8) allows; the
 * device kernels take up to EC_MAX_K data and EC_MAX_M parity shards. */
#define EC_MAX_K 32
#define EC_MAX_M 16

/* A hipStream_t, passed as an opaque pointer so that callers (ctypes, cgo,
 * JNI) need no HIP header. */
typedef void* ec_stream_t;

/* ---- library identity and errors ------------------------------------ */

/* Returns EC_ABI_VERSION of the built library. */
int ec_abi_version(void);

/* Human-readable text for a status code (static storage). */
const char* ec_strerror(int status);

/* ---- host-side GF(2^8) algebra (no device work) ---------------------- */

/* Product of two field elements. */
uint8_t ec_gf_mul(uint8_t a, uint8_t b);

/* Multiplicative inverse; ec_gf_inv(0) returns 0. */
uint8_t ec_gf_inv(uint8_t a);

/* The m x k Cauchy parity block C[i][j] = inv((k+i) ^ j) into out[m*k].
 * Replaces the fixed replica placement of the replication strategy built at
 * megatron/training/training.py:825-828 with an m-of-(k+m) code. */
int ec_cauchy_matrix(int k, int m, uint8_t* out);

/* Gauss-Jordan inverse of the n x n matrix `in` into `out`.
 * EC_ESINGULAR if it is not invertible. */
int ec_gf_invert(const uint8_t* in, uint8_t* out, int n);

/* Decode plan for the code [I_k ; coeff] (coeff is m x k) when the shard
 * indices erased[0..n_erased) of the k+m shards are lost (data shards are
 * 0..k-1, parity shards k..k+m-1).  Writes the k surviving shard indices
 * used (ascending, the first k not erased) to survivors[k] and the
 * n_erased x k matrix rows[] with lost_e = XOR_s rows[e][s] * survivor_s.
 * Serves the load path at megatron/training/checkpointing.py:891-894.
 * EC_ESINGULAR when n_erased > m. */
int ec_decode_matrix(const uint8_t* coeff, int k, int m, const int* erased,
                     int n_erased, int* survivors, uint8_t* rows);

/* ---- device kernels --------------------------------------------------- */

/* XOR parity: d_parity[b] = XOR_{j<k} d_data[j][b].  d_data is a host array
 * of k device pointers.  Any alignment: the bytes from the outputs' first
 * 16-byte boundary on take a vector path when all outputs share one
 * misalignment modulo 16 (inputs realigned as needed); outputs at different
 * misalignments take the byte path throughout.  The same holds for
 * ec_rs_encode and ec_rs_decode.  nbytes = 0 returns
 * EC_OK without touching the shard pointers (empty tensors may have null
 * addresses); so do those two.  Serves manager.save at
 * checkpointing.py:538-541 for m = 1. */
int ec_xor_encode(const uint8_t* const* d_data, int k, uint8_t* d_parity,
                  uint64_t nbytes, ec_stream_t stream);

/* Reed-Solomon encode: d_parity[i][b] = XOR_j coeff[i*k+j] * d_data[j][b].
 * coeff is any m x k host matrix (normally ec_cauchy_matrix).  Serves
 * manager.save at checkpointing.py:538-541. */
int ec_rs_encode(const uint8_t* coeff, int k, int m,
                 const uint8_t* const* d_data, uint8_t* const* d_parity,
                 uint64_t nbytes, ec_stream_t stream);

/* Reconstruct e lost shards from k survivors with the rows computed by
 * ec_decode_matrix: d_out[r][b] = XOR_s rows[r*k+s] * d_survivors[s][b].
 * Serves manager.load at checkpointing.py:891-894. */
int ec_rs_decode(const uint8_t* rows, int k, int e,
                 const uint8_t* const* d_survivors, uint8_t* const* d_out,
                 uint64_t nbytes, ec_stream_t stream);

/* Batched ragged encode: one call over n_stripes stripes of k units of
 * unit_bytes each (one kernel launch on `stream`; two for k = 8, m = 2 over
 * units of 2 MiB up to 16 MiB, which code disjoint tiles).  Device arrays,
 * row-major:
 *   d_data_ptrs[s*k + j]   device address of unit j of stripe s (0 = absent)
 *   d_data_len[s*k + j]    valid bytes of that unit (<= unit_bytes); the
 *                          rest of the unit is taken as zeros
 *   d_parity_ptrs[s*m + i] device address of parity unit i (unit_bytes)
 * The arrays are dense: the kernels read every entry of a stripe, also the
 * length of an absent unit (ignored).
 * unit_bytes must be a multiple of 16 (EC_EALIGN otherwise) and at most
 * 2 GiB (EC_ERANGE).  Units and
 * parity units at 16-byte-aligned addresses take the vector path; others are
 * read and written byte by byte, and no byte past a unit's valid length is
 * read.  Units of 4 KiB and up stream at HBM rate; smaller units work but
 * run a slower byte-granular path.  k <= EC_MAX_K and m <= EC_MAX_M
 * (EC_ERANGE otherwise); k <= 16, m <= 4 run fully unrolled kernels, wider
 * codes a kernel with k at run time.  The units come from the ragged
 * shard list of tensor_aware_state_dict.py:179-184 (MCoreTensorAwareStateDict
 * .tensors), chunked in order. */
int ec_encode_batched(const uint8_t* coeff, int k, int m,
                      const uint64_t* d_data_ptrs, const uint32_t* d_data_len,
                      const uint64_t* d_parity_ptrs, uint32_t n_stripes,
                      uint32_t unit_bytes, ec_stream_t stream);

/* ec_encode_batched, and in the same pass a copy of every data unit:
 * unit (s, j) is written, zero-padded to unit_bytes, at d_copy_ptrs[s*k + j]
 * (0 = no copy of that unit).  The data is read once for the parity and the
 * copy, so coding a checkpoint into one contiguous block (the data units as
 * the block's first k rows, the parity as its last m) costs one pass over
 * HBM.  Copies must not overlap the inputs or the parity.  Same limits and
 * alignment rules as ec_encode_batched (16-byte aligned copies take the fast
 * path); k > 16 or m > 4 runs the encode and the copies as two launches.
 * Serves manager.save at checkpointing.py:538-541: the snapshot of the
 * tensors of tensor_aware_state_dict.py:179-184 that training may overwrite
 * as soon as the call's work has run. */
int ec_encode_batched_copy(const uint8_t* coeff, int k, int m,
                           const uint64_t* d_data_ptrs, const uint32_t* d_data_len,
                           const uint64_t* d_parity_ptrs, const uint64_t* d_copy_ptrs,
                           uint32_t n_stripes, uint32_t unit_bytes, ec_stream_t stream);

/* Batched reconstruct: the stripes of an ec_encode_batched layout that lost
 * the same e shard positions, recovered in one launch with the rows of
 * ec_decode_matrix (e x k):
 *   out_r = XOR_s rows[r*k+s] * survivor_s      for each stripe
 *   d_surv_ptrs[s*k + t], d_surv_len[s*k + t]   the k surviving units of
 *                                               stripe s (data or parity;
 *                                               bytes past len read as zero)
 *   d_out_ptrs[s*e + r], d_out_len[s*e + r]     where lost unit r goes and how
 *                                               many of its bytes to write
 *                                               (a data unit's valid length,
 *                                               so a tensor's tail unit is
 *                                               restored in place without
 *                                               writing past its end)
 * Same alignment rules and limits as ec_encode_batched (e <= EC_MAX_M).  Serves
 * manager.load at checkpointing.py:891-894 for ragged shard lists. */
int ec_decode_batched(const uint8_t* rows, int k, int e,
                      const uint64_t* d_surv_ptrs, const uint32_t* d_surv_len,
                      const uint64_t* d_out_ptrs, const uint32_t* d_out_len,
                      uint32_t n_stripes, uint32_t unit_bytes,
                      ec_stream_t stream);

/* Incremental parity update over n_stripes changed stripes:
 *   parity_i ^= XOR_j coeff[i*k+j] * (new_j ^ old_j)
 * for every unit j whose d_new_ptrs[s*k+j] is non-zero (0 = unchanged unit,
 * skipped).  d_old_ptrs holds the previous contents of the same units and
 * d_len their valid bytes (dense arrays, as in ec_encode_batched: the entries
 * of unchanged units are read and ignored); d_parity_ptrs as in
 * ec_encode_batched.  Stripes
 * must be distinct (each parity unit is read-modified-written by one
 * workgroup).  Same alignment rules and limits as ec_encode_batched.  Serves repeated
 * manager.save calls (checkpointing.py:538-541) when only part of the state
 * changed since the previous checkpoint: a save that names its changed
 * tensors folds them into the coded block the last save left in HBM (old =
 * that block's copy of each unit, parity = its parity units). */
int ec_parity_update(const uint8_t* coeff, int k, int m,
                     const uint64_t* d_new_ptrs, const uint64_t* d_old_ptrs,
                     const uint32_t* d_len, const uint64_t* d_parity_ptrs,
                     uint32_t n_stripes, uint32_t unit_bytes,
                     ec_stream_t stream);

/* ---- a stream for checkpoint work beside training --------------------- */

/* Creates a stream on `device` with a hardware queue of its own, at the
 * default priority: a stream created with a CU mask gets a new queue from the
 * HIP runtime, while plain streams (torch's pooled ones among them) share at
 * most GPU_MAX_HW_QUEUES queues round robin, and two streams on one queue run
 * one after the other.  Measured on MI355X with an 8192^3 bf16 GEMM loop on
 * torch's stream: an RS(6,3) encode beside it on a pooled torch stream that
 * had landed on torch's queue slowed the GEMM by 45 % (the two serialized),
 * on this stream by about 1 %, the
 * encode keeping its full rate.  Kernels only: host<->device copies issued
 * on such a stream held the host and slowed the kernels beside them up to
 * tenfold in the same measurements (on ordinary streams they did not).  The
 * mask holds the first n_cus CUs
 * (n_cus <= 0 or at least the device's CU count: all of them; fewer CUs lower
 * the encode's rate in proportion).  *out receives the stream; release it
 * with ec_stream_destroy.  No counterpart in the reference, whose staging
 * runs in the training process before its async writer starts
 * (megatron/core/dist_checkpointing/strategies/async_utils.py:187-191): this
 * is the stream on which encode and staging run beside train_step
 * (megatron/training/training.py:2316). */
int ec_stream_create(int device, int n_cus, ec_stream_t* out);

/* Waits for the stream's work and destroys it. */
int ec_stream_destroy(ec_stream_t stream);

/* Copies a rows x row_bytes region of device memory (row pitch src_pitch)
 * to host memory that need not be pinned (row pitch dst_pitch), through the
 * caller's pinned buffer h_pinned of pinned_bytes: the buffer's two halves
 * alternate, the transfer of one chunk of columns (one copy per row) runs
 * while `threads` host threads copy the previous chunk out of the other
 * half.  Returns when every byte is in h_dst.  As in
 * ec_stage_stripes_to_host, the copies run on an SDMA engine after the
 * call has waited on the host for the work already enqueued on `stream`
 * when d_src and h_pinned were allocated through the runtime
 * (ec_stage_stats.copy_engine = 1), else as HIP transfers on `stream`,
 * after its work.  EC_EINVAL for null pointers, pitches below
 * row_bytes, threads outside [1, 64], a pinned buffer without room for one
 * byte of every row per half, a region whose size overflows 64 bits, or a
 * runtime allocation holding d_src that ends before the region does; rows
 * or row_bytes 0 is a no-op.  No
 * counterpart in the reference: its checkpoint D2H is
 * copy_tensors_to_cpu (tensor_aware_state_dict.py:245-274), run in the
 * training process before the async writer starts.  The whole loop runs
 * inside the library (a Python caller through ctypes holds no interpreter
 * lock meanwhile).  Pass an ordinary stream, not one from ec_stream_create:
 * measured on MI355X, HIP transfers issued on a CU-masked stream held the
 * host and slowed the kernels beside them. */
int ec_stage_to_host(const uint8_t* d_src, uint64_t src_pitch, uint8_t* h_dst,
                     uint64_t dst_pitch, uint32_t rows, uint64_t row_bytes, uint8_t* h_pinned,
                     uint64_t pinned_bytes, int threads, ec_stream_t stream);

/* Copies a stripe-major device block of n_stripes x positions units of
 * unit_bytes (unit (s, p) at d_block + (s * positions + p) * unit_bytes) to
 * one host row per position: unit (s, p) goes to h_rows[p] + s * unit_bytes,
 * so row p receives position p of every stripe, back to back (n_stripes *
 * unit_bytes bytes; need not be pinned).  The block moves in contiguous
 * chunks of half the caller's pinned buffer while `threads` host threads
 * scatter the previous chunk's units into the rows.  Returns when every
 * byte is in its row.  When d_block and h_pinned were allocated through
 * the runtime (hipMalloc and hipHostMalloc, or torch's allocators over
 * them), each chunk is one copy on an SDMA engine of the GPU, which does
 * not follow streams: the call first waits, on the host, for the work
 * already enqueued on `stream` (the coding of the block), then copies
 * (ec_stage_stats.copy_engine = 1).  Otherwise each chunk is one HIP
 * transfer on `stream`, after its work (copy_engine = 0).  EC_EINVAL for
 * null pointers (any h_rows[p] included), threads outside [1, 64], a
 * pinned buffer under 2 bytes, a block size that overflows 64 bits, or a
 * runtime allocation holding d_block that ends before the block does;
 * n_stripes, positions or unit_bytes 0 is a no-op.  Measured on MI355X
 * beside a training loop (6.44 GB staged every 10 steps of 32 ms): 6-13 ms
 * per save with the engine against 8-82 ms with HIP transfers, which run
 * as copy kernels on one of a few hardware queues, in some runs training's
 * own; the link rate is the same (config 5's 27.4 GB block in 0.49 s).
 * No counterpart in the reference (as for ec_stage_to_host: its checkpoint
 * D2H is copy_tensors_to_cpu, tensor_aware_state_dict.py:245-274).  This is
 * the staging of the block ec_encode_batched_copy writes stripe-major: there
 * the k + m output units of a stripe are adjacent in HBM, which that kernel
 * writes measurably faster than k + m rows each S units long (on MI355X,
 * RS(12,4) over 26,266 stripes of 64 KiB units: 0.79 against 0.74 of the
 * HBM roofline). */
int ec_stage_stripes_to_host(const uint8_t* d_block, uint32_t n_stripes, uint32_t positions,
                             uint64_t unit_bytes, uint8_t* const* h_rows, uint8_t* h_pinned,
                             uint64_t pinned_bytes, int threads, ec_stream_t stream);

/* The way back: row r of a rows x row_bytes region, read from the host
 * array h_rows[r] (need not be pinned; a host array of row_bytes bytes
 * each), goes to d_dst + r * dst_pitch in device memory, through the
 * caller's pinned buffer (two halves: `threads` host threads fill one while
 * the other's transfer runs on `stream`).  Returns when every byte is in
 * device memory; the transfers follow the work already enqueued on
 * `stream`.  Same argument rules as ec_stage_to_host (and null rows are
 * EC_EINVAL).  No counterpart in the reference: its H2D is
 * restore_tensor_device (tensor_aware_state_dict.py:245-274); this call
 * brings the k slices a rank read back into HBM for the decode of
 * manager.load (checkpointing.py:891-894). */
int ec_stage_to_device(const uint8_t* const* h_rows, uint32_t rows, uint64_t row_bytes,
                       uint8_t* d_dst, uint64_t dst_pitch, uint8_t* h_pinned,
                       uint64_t pinned_bytes, int threads, ec_stream_t stream);

/* Timings of a staging call, to tell a slow link from a slow host side. */
typedef struct {
  uint32_t chunks;    /* transfers of one pinned half each                   */
  uint32_t copy_engine; /* 1: the transfers ran on an SDMA engine, 0: HIP    */
  double wall_s;      /* the whole call                                      */
  double wait_s;      /* host time blocked until a half's transfers landed   */
  double host_copy_s; /* host time in the threads' copies (scatter, gather)  */
  double max_wait_s;  /* the longest single wait                             */
  double device_s;    /* device time from the first transfer's start to the
                         last one's end (0 when not measured; with the copy
                         engine, host time from the first copy's start to
                         the last one's landing)                             */
} ec_stage_stats;

/* The timings of the calling thread's last ec_stage_to_host,
 * ec_stage_stripes_to_host or ec_stage_to_device call that moved bytes
 * (kept per thread: the one piece of state the library holds).  EC_EINVAL
 * for a null pointer.  No counterpart in the reference: a diagnostic of the
 * staging of coded checkpoints (tensor_aware_state_dict.py:245-274 is the
 * reference's unmeasured D2H). */
int ec_stage_last_stats(ec_stage_stats* out);

#ifdef __cplusplus
}
#endif

#endif /* EC_MI355_H */
