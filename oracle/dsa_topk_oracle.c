/* dsa_topk_oracle.c - CPU restatement of the DSA top-k page-table transform.
 * TEST INFRASTRUCTURE ONLY: used by tests/ and bench.py's cpu_baseline leg
 * as the checker.
 *
 * Restates the reference's generic path
 * (src/task02_dsa_topk_page_table_transform.py:154-175, the
 * single-program kernel; the chunked path :177-216 computes the same
 * function) and its specification (reports/task02_...md:21-28):
 *
 *   row = (b * H + h) * Q + q
 *   pos = q_pos[b * Q + q], kv_len = kv_lens[b]
 *   valid_blocks = min(ceil(kv_len / block_size), NB)
 *   last_block   = min(pos / block_size, valid_blocks - 1)
 *   block j is selectable iff pos >= 0, j <= last_block and the score
 *   (as fp32) is not -inf
 *   order: score descending (fp32 comparison, so -0 == +0), then block id
 *   ascending
 *   out_blocks[row, t] = t-th selectable block id, or -1 past the count
 *   out_pages[row, t]  = page_table[b * NB + id], or -1
 *
 * Scores are fp32 or bf16 (bits widened to fp32).  NaN scores are outside
 * the contract (the reference's comparison network does not order them).
 * Non-negative kv_len and block_size >= 1 are required.
 */
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define ORC_API __attribute__((visibility("default")))

typedef struct {
  float v;
  int32_t id;
} cand_t;

static int better(const cand_t* a, const cand_t* b) {
  if (a->v > b->v) return 1;
  if (a->v < b->v) return 0;
  return a->id < b->id;
}

static int cmp_cand(const void* pa, const void* pb) {
  const cand_t* a = (const cand_t*)pa;
  const cand_t* b = (const cand_t*)pb;
  if (better(a, b)) return -1;
  if (better(b, a)) return 1;
  return 0;
}

static float score_at(const void* scores, int bf16, int64_t i) {
  if (bf16) {
    const uint32_t u = (uint32_t)((const uint16_t*)scores)[i] << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
  }
  return ((const float*)scores)[i];
}

static int64_t index_at(const void* p, int idx64, int64_t i) {
  return idx64 ? ((const int64_t*)p)[i] : (int64_t)((const int32_t*)p)[i];
}

/* scores [B, H, Q, NB] (fp32, or bf16 bits when scores_bf16); page_table
 * int32 [B, NB]; q_pos [B, Q] and kv_lens [B], int32 or int64 (index64);
 * out_blocks, out_pages int32 [B, H, Q, top_k].  Returns 0, or 1 on an
 * argument outside the contract. */
ORC_API int orc_dsa_topk(const void* scores, int scores_bf16, const int32_t* page_table,
                         const void* q_pos, const void* kv_lens, int index64,
                         int32_t* out_blocks, int32_t* out_pages, int64_t B, int64_t H,
                         int64_t Q, int64_t NB, int64_t block_size, int64_t top_k,
                         int nthreads) {
  if (B < 0 || H < 0 || Q < 0 || NB <= 0 || block_size < 1 || top_k < 1) return 1;
  const int64_t rows = B * H * Q;
  int fail = 0;
#pragma omp parallel num_threads(nthreads > 0 ? nthreads : 1) if (rows > 1)
  {
    cand_t* c = (cand_t*)malloc((size_t)NB * sizeof(cand_t));
    if (!c) {
#pragma omp atomic write
      fail = 1;
    } else {
#pragma omp for schedule(static)
      for (int64_t row = 0; row < rows; ++row) {
        const int64_t q = row % Q;
        const int64_t b = (row / Q) / H;
        const int64_t pos = index_at(q_pos, index64, b * Q + q);
        const int64_t kv_len = index_at(kv_lens, index64, b);
        int64_t valid_blocks = (kv_len + block_size - 1) / block_size;
        if (valid_blocks > NB) valid_blocks = NB;
        int64_t last = pos / block_size;
        if (last > valid_blocks - 1) last = valid_blocks - 1;
        int64_t n = 0;
        if (pos >= 0) {
          for (int64_t j = 0; j <= last && j < NB; ++j) {
            const float v = score_at(scores, scores_bf16, row * NB + j);
            if (v == -__builtin_inff()) continue;
            c[n].v = v;
            c[n].id = (int32_t)j;
            ++n;
          }
        }
        qsort(c, (size_t)n, sizeof(cand_t), cmp_cand);
        for (int64_t t = 0; t < top_k; ++t) {
          if (t < n) {
            out_blocks[row * top_k + t] = c[t].id;
            out_pages[row * top_k + t] = page_table[b * NB + c[t].id];
          } else {
            out_blocks[row * top_k + t] = -1;
            out_pages[row * top_k + t] = -1;
          }
        }
      }
      free(c);
    }
  }
  return fail;
}
