/*
 * fagq_diag.h - test and measurement entry points of the fagq library.
 *
 * None of these has a counterpart in the reference
 * (sinpeyw/flagos-kernelgen-72h-shanghai-2026); they exist so that tests can
 * exercise every launch mapping, the device number-format encoders and the
 * scale addressing directly.  Same conventions as fagq.h: device pointers,
 * stream-ordered, status codes, no allocation.  The measurement probes (HBM
 * streams, matrix-instruction rate, LDS reads) live in a library of their
 * own, libfagq_probe.so (fagq_probe.h).
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

#ifdef __cplusplus
}
#endif

#endif /* FAGQ_DIAG_H */
