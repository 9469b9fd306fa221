/* fagq_gemm.h - C ABI of the fp8 block-scaled GEMM that consumes the
 * quantizer's output (libfagq.so, gfx950).
 *
 *   C[m, n] = bf16_rne( sum_kb  sa(m, kb) * sb(n / 128, kb) * P_kb[m, n] ),
 *   P_kb[m, n] = sum_{k in block kb} A[m, k] * B[n, k]        (fp8 x fp8, fp32)
 *
 * A is the quantizer's code tensor q [M, K] (fp8 e4m3fn) and sa its per-token
 * 1 x 128 group scales, in the quantizer's column-major ([K/128, M] physical)
 * or row-major ([M, K/128]) layout, fp32 or UE8M0 bytes.  B is a weight
 * [N, K] (fp8 e4m3fn, K contiguous) with one scale per 128 x 128 block,
 * sb [ceil(N/128), K/128] row-major, fp32 or UE8M0.  This is the DeepSeek-V3
 * style fp8 linear layer that the column-major and UE8M0 scale formats of the
 * quantizer exist to feed.
 *
 * No counterpart in the reference repository: the reference's operator
 * (src/task01_fused_add_rmsnorm_group_quant.py:1731-1851) ends at the
 * quantized tensor and its scales; this is the consumer of that wire format.
 *
 * Accumulation is fp32 inside each 128-deep block (the MFMA's own order),
 * then fp32 across blocks in block order.  With both scales UE8M0 the scales
 * are applied by the matrix core itself (exact powers of two).
 *
 * Same conventions as fagq.h: device pointers, stream-ordered, no allocation,
 * no synchronization; returns 0, a FAGQ_E_* code (> 0) or -hipError_t.
 */
#ifndef FAGQ_GEMM_H_
#define FAGQ_GEMM_H_

#include <stdint.h>

#include "fagq.h"

#ifdef __cplusplus
extern "C" {
#endif

/* a_q      fp8 e4m3fn [M, K], rows 16-byte aligned (K % 128 == 0)
 * a_scale  fp32 or uint8 (UE8M0); layout FAGQ_LAYOUT_COL_MAJOR ([K/128, M]
 *          physical) or FAGQ_LAYOUT_ROW_MAJOR ([M, K/128])
 * b_q      fp8 e4m3fn [N, K]
 * b_scale  fp32 or uint8 (UE8M0) [ceil(N/128), K/128] row-major
 * c        bf16 [M, N] row-major, N % 16 == 0
 * a_scale_format, b_scale_format: FAGQ_SCALE_F32 or FAGQ_SCALE_UE8M0 */
FAGQ_API int fagq_gemm_launch(const void* a_q, const void* a_scale, const void* b_q, const void* b_scale,
                              void* c, int64_t M, int64_t N, int64_t K, int a_scale_format,
                              int a_scale_layout, int b_scale_format, void* stream);

/* Launch geometry of fagq_gemm_launch for a shape (no device access). */
typedef struct fagq_gemm_route {
  int32_t block_m;      /* output rows per workgroup */
  int32_t block_n;      /* output columns per workgroup */
  int32_t block_threads;
  int32_t group_m;      /* row tiles per group in the tile order */
  int64_t grid_blocks;
} fagq_gemm_route;

FAGQ_API int fagq_gemm_query_route(int64_t M, int64_t N, int64_t K, fagq_gemm_route* route);

#ifdef __cplusplus
}
#endif

#endif /* FAGQ_GEMM_H_ */
