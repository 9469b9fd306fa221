/* mla_bwd_oracle.c - CPU restatement of the reference's Task 03 operator
 * (MLA backward, NoPE, shared K = V = C).
 * TEST INFRASTRUCTURE ONLY: used by tests/ and bench.py's cpu_baseline leg
 * as the checker.
 *
 * Restates what mla_bwd_nope_dkdv (src/task03_mla_bwd_nope_dkdv.py:453-480)
 * computes on a GPU (_run_gpu, :401-425):
 *   _exact_prefix_reuse_dq_kernel (:137-201), EXACT_ROWS = 16 (:405): for
 *   query rows i < E = min(16, S) of every (b, h), keys j <= i,
 *     delta_i = sum_d out[i, d] do[i, d]
 *     P_ij  = bf16(exp2((q_i . c_j * sm_scale - lse_i) * log2 e))
 *     dS_ij = bf16(P_ij (do_i . c_j - delta_i) sm_scale)
 *     dq_i  = sum_j dS_ij c_j
 *   _uniform_dc_headsum_tiled_kernel (:268-303): dq_i = fp32(do_i) * sm_scale
 *   for rows i >= E, and hs_i = sum_h do[h, i];
 *   _uniform_dc_parallel_scan_kernel (:305-330): dc_j = sum_{i >= j} hs_i / (i + 1).
 * Dot products and sums run in float64 here (the reference accumulates in
 * fp32); P and dS are rounded to fp32 and then to bf16 (round to nearest
 * even), the reference's fp32 -> bf16 casts.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define ORC_API __attribute__((visibility("default")))
#define EXACT_ROWS 16

static double bf(uint16_t h) {
  const uint32_t u = (uint32_t)h << 16;
  float f;
  memcpy(&f, &u, 4);
  return (double)f;
}

/* fp32 -> bf16 -> fp32, round to nearest even (finite inputs). */
static float round_bf16(float x) {
  uint32_t u;
  memcpy(&u, &x, 4);
  u = (u + 0x7fffu + ((u >> 16) & 1u)) & 0xffff0000u;
  float r;
  memcpy(&r, &u, 4);
  return r;
}

/* q, out, dout [B, H, S, D] and c [B, S, D] bf16 bits; lse [B, H, S] fp32.
 * Writes dq [B, H, S, D] and dc [B, S, D] (float64), and, when dq_bound is
 * not NULL, two error scales of the exact rows, [B, H, E, D] each:
 *   dq_bound[0] = sum_j |dS_ij| |c_jd|  (a bf16 step of P or dS moves dq by
 *                 at most 2^-8 of this);
 *   dq_bound[1] = sum_j P_ij sm_scale (sum_d' |do_id'| |c_jd'| + sum_d' |out_id'|
 *                 |do_id'|) |c_jd|  (the sensitivity of dq to absolute
 *                 errors in dp_ij - delta_i, which cancel when out is close
 *                 to the rows of c).
 * Returns 0, or 1 on an argument outside the contract. */
ORC_API int orc_mla_bwd(const uint16_t* q, const uint16_t* c, const uint16_t* out,
                        const uint16_t* dout, const float* lse, double* dq, double* dc,
                        double* dq_bound, int64_t B, int64_t H, int64_t S, int64_t D,
                        float sm_scale, int nthreads) {
  if (B < 0 || H < 1 || S < 1 || D < 1) return 1;
  const int64_t E = S < EXACT_ROWS ? S : EXACT_ROWS;
  const int nt = nthreads > 0 ? nthreads : 1;
#pragma omp parallel for num_threads(nt) schedule(dynamic)
  for (int64_t bh = 0; bh < B * H; ++bh) {
    const int64_t b = bh / H;
    const uint16_t* qb = q + bh * S * D;
    const uint16_t* ob = out + bh * S * D;
    const uint16_t* db = dout + bh * S * D;
    const uint16_t* cb = c + b * S * D;
    double dS[EXACT_ROWS][EXACT_ROWS], sens[EXACT_ROWS][EXACT_ROWS];
    for (int64_t i = 0; i < E; ++i) {
      double delta = 0.0, adelta = 0.0;
      for (int64_t d = 0; d < D; ++d) {
        delta += bf(ob[i * D + d]) * bf(db[i * D + d]);
        adelta += fabs(bf(ob[i * D + d]) * bf(db[i * D + d]));
      }
      for (int64_t j = 0; j < E; ++j) {
        dS[i][j] = sens[i][j] = 0.0;
        if (j > i) continue;
        double logit = 0.0, dp = 0.0, adp = 0.0;
        for (int64_t d = 0; d < D; ++d) {
          logit += bf(qb[i * D + d]) * bf(cb[j * D + d]);
          dp += bf(db[i * D + d]) * bf(cb[j * D + d]);
          adp += fabs(bf(db[i * D + d]) * bf(cb[j * D + d]));
        }
        const double arg = (logit * (double)sm_scale - (double)lse[bh * S + i]) * 1.4426950408889634;
        const float p = round_bf16((float)exp2(arg));
        dS[i][j] = (double)round_bf16((float)((double)p * (dp - delta) * (double)sm_scale));
        sens[i][j] = (double)p * (double)sm_scale * (adp + adelta);
      }
      for (int64_t d = 0; d < D; ++d) {
        double acc = 0.0, bound = 0.0, cbound = 0.0;
        for (int64_t j = 0; j <= i; ++j) {
          acc += dS[i][j] * bf(cb[j * D + d]);
          bound += fabs(dS[i][j]) * fabs(bf(cb[j * D + d]));
          cbound += sens[i][j] * fabs(bf(cb[j * D + d]));
        }
        dq[(bh * S + i) * D + d] = acc;
        if (dq_bound) {
          dq_bound[(bh * E + i) * D + d] = bound;
          dq_bound[B * H * E * D + (bh * E + i) * D + d] = cbound;
        }
      }
    }
    for (int64_t i = E; i < S; ++i)
      for (int64_t d = 0; d < D; ++d)
        dq[(bh * S + i) * D + d] = (double)((float)bf(db[i * D + d]) * sm_scale);
  }
#pragma omp parallel for num_threads(nt) schedule(static)
  for (int64_t bd = 0; bd < B * D; ++bd) {
    const int64_t b = bd / D, d = bd % D;
    double run = 0.0;
    for (int64_t i = S - 1; i >= 0; --i) {
      double hs = 0.0;
      for (int64_t h = 0; h < H; ++h) hs += bf(dout[((b * H + h) * S + i) * D + d]);
      run += hs / (double)(i + 1);
      dc[(b * S + i) * D + d] = run;
    }
  }
  return 0;
}
