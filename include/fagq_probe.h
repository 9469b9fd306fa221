/*
 * fagq_probe.h - measurement probes (libfagq_probe.so): what the machine
 * allows the operators' kernels, measured with kernels of the same shape and
 * cache policies but none of their work.  Not part of the drop-in library
 * (libfagq.so); bench.py's --copy, --mfma-peak and --lds-probe modes and the
 * probe tests load it.  No counterpart in the reference.  Same conventions as
 * fagq.h: device pointers, stream-ordered, status codes (FAGQ_E_*), no
 * allocation.
 */
#ifndef FAGQ_PROBE_H
#define FAGQ_PROBE_H

#include <stdint.h>

#include "fagq.h"

#ifdef __cplusplus
extern "C" {
#endif

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

#endif /* FAGQ_PROBE_H */
