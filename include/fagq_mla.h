/* fagq_mla.h - C ABI of the MLA backward (NoPE, shared K = V = C) gradient
 * dQ and dC (libfagq.so, gfx950): Task 03 of the reference repository.
 *
 * Replaces mla_bwd_nope_dkdv (src/task03_mla_bwd_nope_dkdv.py:453-480), with
 * the function its GPU path computes (_run_gpu, :401-425):
 *
 *   E = min(16, S) query rows per (b, h) get the exact gradient
 *   (_exact_prefix_reuse_dq_kernel, :137-201), keys j <= i:
 *     delta_i = sum_d out[i, d] do[i, d]
 *     P_ij    = bf16(exp2((q_i . c_j * sm_scale - lse_i) * log2 e))
 *     dS_ij   = bf16(P_ij (do_i . c_j - delta_i) sm_scale)
 *     dq_i    = sum_j dS_ij c_j
 *   rows i >= E: dq_i = sm_scale * do_i (:285-297)
 *   dc_j = sum_{i >= j} (sum_h do[h, i]) / (i + 1)   (:269-330), the
 *   uniform-causal dV of reports/task03_mla_bwd_nope_dkdv.md:160-176
 *
 * The exact backward of reports/task03_...md:23-39 is not this function:
 * the reference approximates dq for rows >= E and dc everywhere, and this
 * library reproduces the reference.
 *
 * Same conventions as fagq.h: device pointers, stream-ordered, no
 * allocation (the caller passes a workspace), no synchronization; returns
 * 0, a FAGQ_E_* code or -hipError_t.
 */
#ifndef FAGQ_MLA_H_
#define FAGQ_MLA_H_

#include <stdint.h>

#include "fagq.h"

#ifdef __cplusplus
extern "C" {
#endif

#define FAGQ_MLA_EXACT_ROWS 16
#define FAGQ_MLA_SLICE_D 512

enum fagq_mla_dtype { FAGQ_MLA_F32 = 0, FAGQ_MLA_BF16 = 1 };

/* Workspace bytes fagq_mla_bwd_launch needs for (B, S, D): fp32 partial
 * head sums [G, B, S, W] (G = 1 when the row grid fills the GPU, else up to 8
 * head groups) and the scan's block totals [B, nblk, W] (blocks of 16-64
 * rows), W = min(D, FAGQ_MLA_SLICE_D).  Returns -1 for a negative or
 * overflowing size. */
FAGQ_API int64_t fagq_mla_bwd_workspace_bytes(int64_t B, int64_t S, int64_t D);

/* q [B, H, S, D], out and dout [B, H, S, D], c_kv [B, S, D]: bfloat16,
 * contiguous, 16-byte aligned.  lse [B, H, S] fp32 (natural-log logsumexp
 * of the forward).  dq [B, H, S, D] and dc_kv [B, S, D]: fp32 or bf16
 * (dq_dtype, dc_dtype), 16-byte aligned.  workspace: at least
 * fagq_mla_bwd_workspace_bytes(B, S, D) bytes, 16-byte aligned, overwritten.
 * D >= 64, D % 64 == 0; B, H <= 65535; S >= 1; H * S * D * 4 < 2^32.
 * Three kernels on `stream` per column slice of FAGQ_MLA_SLICE_D dims (one
 * slice for D <= 512; the reference's kernels, src/task03_mla_bwd_nope_dkdv.py:154,
 * 166, 191, likewise walk D in 128-wide chunks with no cap). */
FAGQ_API int fagq_mla_bwd_launch(const void* q, const void* c_kv, const void* out, const void* dout,
                                 const float* lse, void* dq, void* dc_kv, void* workspace,
                                 int64_t workspace_bytes, int64_t B, int64_t H, int64_t S,
                                 int64_t D, float sm_scale, int dq_dtype, int dc_dtype,
                                 void* stream);

/* Scratch bytes fagq_mla_bwd_launch_noalloc holds on each GPU it runs on. */
#define FAGQ_MLA_SCRATCH_BYTES (32ll << 20)

/* fagq_mla_bwd_launch without a workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  No counterpart in the reference: its
 * operator allocates its head-sum buffer per call.  The workspace is a
 * library-owned array of FAGQ_MLA_SCRATCH_BYTES per GPU, created with the
 * library's code on that GPU and held until the process ends; this call
 * allocates nothing.  Calls whose workspace (fagq_mla_bwd_workspace_bytes)
 * exceeds it return FAGQ_E_TOO_LARGE.  Every call on a GPU shares that GPU's
 * array: calls that overlap on one GPU (other streams, or other host threads)
 * race and must be ordered by the caller.  Nothing needs clearing between
 * calls: every workspace word a call reads, the same call has written first.
 * Other arguments and results as fagq_mla_bwd_launch. */
FAGQ_API int fagq_mla_bwd_launch_noalloc(const void* q, const void* c_kv, const void* out,
                                         const void* dout, const float* lse, void* dq,
                                         void* dc_kv, int64_t B, int64_t H, int64_t S, int64_t D,
                                         float sm_scale, int dq_dtype, int dc_dtype,
                                         void* stream);

#ifdef __cplusplus
}
#endif

#endif /* FAGQ_MLA_H_ */
