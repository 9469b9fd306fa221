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
 * ceil(ceil(D / 512) / waves_per_row) <= 16 and, when that exceeds 4,
 * waves_per_row * rows_per_block <= 4; rows_in_sequence in [1, 64] rows
 * per row group, processed in turn.  xcd_remap selects the workgroup ->
 * row-tile order: 0 dispatch order, 1 one contiguous range of tiles per XCD,
 * n in {2, 4, .., 64} chunks of n consecutive tiles per XCD.  Returns
 * FAGQ_E_FORMAT for an invalid mapping. */
FAGQ_API int fagq_launch_mapped(const void* x, const void* residual, const void* gamma,
                                void* residual_out, void* norm_out, void* q, void* scale,
                                int64_t M, int64_t D, int64_t group_size, float eps,
                                int q_format, int scale_format, int scale_layout,
                                int rounding, int waves_per_row, int rows_per_block,
                                int rows_in_sequence, int xcd_remap, void* stream);

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
 * device encoder, after a clamp to [-QMAX, QMAX] (which the operator itself
 * never needs: its values are within that range): one byte per value. */
FAGQ_API int fagq_diag_encode(const float* in, void* out, int64_t n, int q_format,
                              int rounding, void* stream);

/* Copies `bytes` (a multiple of 16, both pointers 16-byte aligned) with a
 * plain 16-byte-vector streaming kernel. */
FAGQ_API int fagq_diag_copy(const void* src, void* dst, int64_t bytes, void* stream);

/* Issue-rate probe of the fp8 GEMM's matrix instruction: `blocks`
 * workgroups of 4 waves (1 <= blocks <= 2^20), each wave issuing iters x 8
 * v_mfma_scale_f32_16x16x128_f8f6f4 (1 <= iters <= 2^20) on register
 * operands with no memory traffic, then writing one float per thread:
 * `out` holds blocks x 256 floats.  One launch performs
 * blocks x 4 x iters x 8 x 65536 flops, the ceiling the GEMM's measured
 * rate is compared with. */
FAGQ_API int fagq_diag_mfma_peak(float* out, int64_t blocks, int32_t iters, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* FAGQ_DIAG_H */
