/*
 * fagq_diag.h - test and measurement entry points of the fagq library.
 *
 * None of these has a counterpart in the reference
 * (sinpeyw/flagos-kernelgen-72h-shanghai-2026); they exist so that tests can
 * exercise every launch mapping and the device number-format encoders
 * directly, and so that HBM byte counters can be calibrated against a copy
 * of known size.  Same conventions as fagq.h: device pointers,
 * stream-ordered, status codes, no allocation.
 */
#ifndef FAGQ_DIAG_H
#define FAGQ_DIAG_H

#include <stdint.h>

#include "fagq.h"

#ifdef __cplusplus
extern "C" {
#endif

/* fagq_launch with an explicit mapping instead of the route table:
 * waves_per_row in [1, 16], rows_per_block >= 1 with
 * waves_per_row * rows_per_block <= 16, steps per wave
 * ceil(ceil(D / 512) / waves_per_row) <= 4.  row_group_mode: 0 independent
 * rows; 1 gamma loaded by the workgroup's first row and shared through LDS;
 * 2 as 1, and the first row's waves store each group's column-major scales of
 * all rows_per_block rows with one store (column-major scales only,
 * rows_per_block 2 or 4).  Modes 1 and 2 need
 * waves_per_row * steps per wave <= 16 (D <= 8192).  xcd_remap selects the
 * workgroup -> row-tile order: 0 dispatch order, 1 one contiguous range of
 * tiles per XCD, n in {2, 4, .., 64} chunks of n consecutive tiles per XCD.
 * lds_bytes in [0, 65536] of dynamic LDS is reserved per workgroup (the kernel
 * does not use it; it caps the workgroups resident per CU).  Every mapping
 * gives the same bits.  Returns FAGQ_E_FORMAT for an invalid mapping. */
FAGQ_API int fagq_launch_mapped(const void* x, const void* residual, const void* gamma,
                                void* residual_out, void* norm_out, void* q, void* scale,
                                int64_t M, int64_t D, int64_t group_size, float eps,
                                int q_format, int scale_format, int scale_layout,
                                int rounding, int waves_per_row, int rows_per_block,
                                int row_group_mode, int xcd_remap, int lds_bytes, void* stream);

/* fagq_gemm_launch with the tile width forced: block_n 192 or 256 columns
 * of C per workgroup (0: the shape's own choice, as fagq_gemm_launch).  Any
 * width gives the same bits: each output takes the same MFMA and scale
 * sequence.  Other arguments and rules as fagq_gemm_launch (fagq_gemm.h);
 * FAGQ_E_FORMAT for another block_n. */
FAGQ_API int fagq_gemm_launch_mapped(const void* a_q, const void* a_scale, const void* b_q,
                                     const void* b_scale, void* c, int64_t M, int64_t N,
                                     int64_t K, int a_scale_format, int a_scale_layout,
                                     int b_scale_format, int block_n, void* stream);

/* Encodes n fp32 values (n % 8 == 0, 16-byte aligned) with the operator's
 * device encoder: one byte per value.  clamp = 1 applies the reference's
 * clamp to [-QMAX, QMAX] first; clamp = 0 passes the values unclamped, as the
 * operator's kernels do (their values stay below QMAX * (1 + 5 * 2^-24)). */
FAGQ_API int fagq_diag_encode(const float* in, void* out, int64_t n, int q_format,
                              int rounding, int clamp, void* stream);

/* HBM ceiling probes with the operator's cache policies (non-temporal loads,
 * sc1 | nt stores), one 16-byte chunk per thread, 512 threads per
 * workgroup.  `bytes` is a multiple of 16, pointers 16-byte aligned.
 *   FAGQ_STREAM_COPY   reads src, writes dst (bytes each)
 *   FAGQ_STREAM_READ   reads src; dst (>= 16 bytes) is written only if a
 *                      chunk's four words XOR to 0x9e3779b9
 *   FAGQ_STREAM_WRITE  writes dst; src may be NULL
 *   FAGQ_STREAM_OPMIX  the operator's byte mix without its arithmetic: reads
 *                      src[0, bytes) and src[bytes, 2 bytes) (x and residual),
 *                      writes dst[0, bytes) and dst[bytes, 1.5 bytes)
 *                      (residual_out and one-byte codes); src holds 2 bytes,
 *                      dst 1.5 bytes, bytes a multiple of 32 */
enum fagq_stream_mode {
  FAGQ_STREAM_COPY = 0,
  FAGQ_STREAM_READ = 1,
  FAGQ_STREAM_WRITE = 2,
  FAGQ_STREAM_OPMIX = 3
};

FAGQ_API int fagq_diag_stream(const void* src, void* dst, int64_t bytes, int mode, void* stream);

/* fagq_diag_stream(src, dst, bytes, FAGQ_STREAM_COPY, stream): the copy of
 * known size that HBM byte counters are calibrated against. */
FAGQ_API int fagq_diag_copy(const void* src, void* dst, int64_t bytes, void* stream);

/* Host-side check of the operator's per-lane scale addressing, computed by
 * the same functions the kernels use: for row `row` of an [M, D] call split
 * over waves_per_row waves (one row per workgroup), writes for every wave,
 * step and lane out[(wave * steps_per_wave + step) * 64 + lane] = the scale
 * element index that lane's store reaches, or -1 when the buffer descriptor
 * drops it.  cap >= waves_per_row * steps_per_wave * 64.  Never touches the
 * device. */
FAGQ_API int fagq_diag_scale_offsets(int64_t M, int64_t D, int64_t group_size, int scale_format,
                                     int scale_layout, int waves_per_row, int64_t row,
                                     int64_t* out, int64_t cap);

/* Issue-rate probe of the fp8 GEMM's matrix instruction: `blocks`
 * workgroups of 4 waves (1 <= blocks <= 2^20), each wave issuing iters x 8
 * v_mfma_scale_f32_16x16x128_f8f6f4 (1 <= iters <= 2^20) on register
 * operands with no memory traffic, then writing one float per thread:
 * `out` holds blocks x 256 floats.  One launch performs
 * blocks x 4 x iters x 8 x 65536 flops, the ceiling the GEMM's measured
 * rate is compared with. */
FAGQ_API int fagq_diag_mfma_peak(float* out, int64_t blocks, int32_t iters, void* stream);

/* The same probe for either fp8 matrix-instruction shape: shape 0 is
 * fagq_diag_mfma_peak; shape 1 issues iters x 4
 * v_mfma_scale_f32_32x32x64_f8f6f4 per wave (4 independent 32 x 32
 * accumulators), blocks x 4 x iters x 4 x 131072 flops per launch. */
FAGQ_API int fagq_diag_mfma_rate(float* out, int64_t blocks, int32_t iters, int shape,
                                 void* stream);

/* LDS bank probe of the GEMM's operand reads: `blocks` workgroups of 4
 * waves (1 <= blocks <= 2^20); every lane reads 16 bytes with ds_read_b128,
 * 8 x iters times (1 <= iters <= 2^20), from 16 KB of LDS holding 32-bit
 * word i = i * 0x9E3779B1 (mod 2^32), at byte address
 *   pattern 0: 16 (l % 64)                              (1 KB in lane order)
 *   pattern 1: 128 r + 16 (c ^ f(r)),  f(r) = ((r >> 1) & 1) | (r & 4)
 *   pattern 2: as 1 with c + 1 for c                    (the GEMM's swizzle)
 *   pattern 3: 128 r + 16 (c ^ ((r >> 1) & 7))
 *   pattern 4: 128 r + 16 (c ^ (r & 7))
 *   pattern 5: 128 r + 16 c                             (no swizzle)
 * with r = l % 16 and c = 2 ((l % 64) / 16) for thread l, and writes the 4
 * words it read: `out` holds blocks x 256 x 4 int32 (16-byte aligned).
 * Bank conflicts show in rocprofv3's SQ_LDS_BANK_CONFLICT per SQ_INSTS_LDS. */
FAGQ_API int fagq_diag_lds_read(int32_t* out, int64_t blocks, int32_t iters, int pattern,
                                void* stream);

#ifdef __cplusplus
}
#endif

#endif /* FAGQ_DIAG_H */
