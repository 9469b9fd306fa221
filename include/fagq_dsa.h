/* fagq_dsa.h - C ABI of the DSA top-k page-table transform (libfagq.so,
 * gfx950): Task 02 of the reference repository.
 *
 * Replaces dsa_topk_page_table_transform
 * (src/task02_dsa_topk_page_table_transform.py:1666-1726, semantics of its
 * generic path :154-175; reports/task02_dsa_topk_page_table_transform.md:21-28):
 *
 *   for row (b, h, q) of scores[B, H, Q, NB]:
 *     pos = q_pos[b, q], kv_len = kv_lens[b]
 *     valid_blocks = min(ceil(kv_len / block_size), NB)
 *     last_block   = min(pos / block_size, valid_blocks - 1)
 *     block j is selectable iff pos >= 0, j <= last_block, score != -inf
 *     order: score descending (fp32 compare, -0 == +0), then block id ascending
 *     out_blocks[b, h, q, t] = t-th selectable id, or -1 past their count
 *     out_pages[b, h, q, t]  = page_table[b, id], or -1
 *
 * Scores: fp32 or bf16 (compared as fp32), no NaN.  kv_lens >= 0.
 * Same conventions as fagq.h: device pointers, stream-ordered, no
 * allocation, no synchronization; returns 0, a FAGQ_E_* code or
 * -hipError_t.
 */
#ifndef FAGQ_DSA_H_
#define FAGQ_DSA_H_

#include <stdint.h>

#include "fagq.h"

#ifdef __cplusplus
extern "C" {
#endif

#define FAGQ_DSA_MAX_NB (1 << 28)
#define FAGQ_DSA_MAX_TOP_K 1024

enum fagq_dsa_scores { FAGQ_DSA_F32 = 0, FAGQ_DSA_BF16 = 1 };
enum fagq_dsa_index { FAGQ_DSA_I32 = 0, FAGQ_DSA_I64 = 1 };

/* scores      [B, H, Q, NB] fp32 or bf16 (scores_dtype), aligned to its element
 *             size (rows read as 16-byte vectors when the pointer is 16-byte
 *             aligned and NB * element size is a multiple of 16, else one score
 *             per load)
 * page_table  int32 [B, NB]
 * q_pos       [B, Q], kv_lens [B]: int32 or int64 (index_dtype)
 * out_blocks, out_pages  int32 [B, H, Q, top_k]
 * 1 <= NB <= FAGQ_DSA_MAX_NB, 1 <= top_k <= FAGQ_DSA_MAX_TOP_K, 1 <= block_size < 2^31,
 * B and H <= 65535, B * H * Q < 2^31, Q * 64 * min(16, ceil(NB / 1024)) < 2^32
 * (FAGQ_E_TOO_LARGE otherwise) */
FAGQ_API int fagq_dsa_topk_launch(const void* scores, int scores_dtype, const void* page_table,
                                  const void* q_pos, const void* kv_lens, int index_dtype,
                                  void* out_blocks, void* out_pages, int64_t B, int64_t H,
                                  int64_t Q, int64_t NB, int64_t block_size, int64_t top_k,
                                  void* stream);

#ifdef __cplusplus
}
#endif

#endif /* FAGQ_DSA_H_ */
