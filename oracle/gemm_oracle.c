/* gemm_oracle.c - CPU restatement of the fp8 block-scaled GEMM that consumes
 * the quantizer's output (include/fagq_gemm.h).  TEST INFRASTRUCTURE ONLY:
 * used by tests/ and bench.py's cpu_baseline leg as the checker.
 *
 * No counterpart in the reference repository: its operator
 * (src/task01_fused_add_rmsnorm_group_quant.py:1731-1851) stops at the
 * quantized tensor and scales; this restates the consumer those formats feed
 * (a DeepSeek-V3 style 1 x 128 / 128 x 128 block-scaled fp8 linear layer):
 *
 *   C[m, n] = sum_kb s(m, n, kb) * P_kb[m, n],   s = fp32(sa(m, kb) * sb(n / 128, kb))
 *   P_kb[m, n] = sum_{k in block kb} A[m, k] * B[n, k]
 *
 * Each fp8 e4m3fn value has a 4-bit significand and exponents in
 * [2^-9, 2^8], so every product is exact in double and a 128-term block sum
 * spans at most 2^-18 .. 2^24: exact in double too.  P_kb is therefore exact;
 * s * P_kb and the sum over blocks are rounded in double.  The function also
 * returns, per element, sum_kb |s| * sum_k |A B|, which bounds the rounding
 * error of any fp32 evaluation order.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

#define ORC_API __attribute__((visibility("default")))

/* e4m3fn (OCP): sign, 4-bit exponent (bias 7), 3-bit mantissa, no inf;
 * S.1111.111 is NaN; exponent 0 is subnormal: m * 2^-9. */
static double e4m3fn_to_f64(uint8_t b) {
  const int s = b >> 7, e = (b >> 3) & 15, m = b & 7;
  double v;
  if (e == 15 && m == 7) return NAN;
  if (e == 0)
    v = ldexp((double)m, -9);
  else
    v = ldexp((double)(8 + m), e - 10);   /* (1 + m/8) * 2^(e-7) */
  return s ? -v : v;
}

ORC_API void orc_e4m3fn_to_f64(const uint8_t* in, double* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = e4m3fn_to_f64(in[i]);
}

static float e8m0_to_f32(uint8_t e) { return ldexpf(1.0f, (int)e - 127); }

static float scale_at(const void* p, int fmt, int64_t idx) {
  if (fmt == 0) {
    float f;
    memcpy(&f, (const uint8_t*)p + 4 * idx, 4);
    return f;
  }
  return e8m0_to_f32(((const uint8_t*)p)[idx]);
}

/* a_q [M, K], b_q [N, K] (fp8 bits); a_scale [M, K/128] row-major
 * (a_layout 0) or [K/128, M] (a_layout 1); b_scale [ceil(N/128), K/128];
 * formats 0 = fp32, 1 = UE8M0.  c, cabs: double [M, N].  Returns 0, or 2 for
 * a shape it does not accept. */
ORC_API int orc_gemm(const uint8_t* a_q, const void* a_scale, const uint8_t* b_q,
                     const void* b_scale, double* c, double* cabs, int64_t M, int64_t N,
                     int64_t K, int a_fmt, int a_layout, int b_fmt, int nthreads) {
  if (M < 0 || N <= 0 || K <= 0 || K % 128 != 0) return 2;
  const int64_t KB = K / 128;
  if (nthreads <= 0) nthreads = 1;
#pragma omp parallel for schedule(static) num_threads(nthreads)
  for (int64_t m = 0; m < M; ++m) {
    double arow[128];
    for (int64_t n = 0; n < N; ++n) {
      double acc = 0.0, accabs = 0.0;
      for (int64_t kb = 0; kb < KB; ++kb) {
        const float sa = scale_at(a_scale, a_fmt, a_layout ? kb * M + m : m * KB + kb);
        const float sb = scale_at(b_scale, b_fmt, (n / 128) * KB + kb);
        const float s = sa * sb;
        for (int k = 0; k < 128; ++k) arow[k] = e4m3fn_to_f64(a_q[m * K + kb * 128 + k]);
        double p = 0.0, pabs = 0.0;
        for (int k = 0; k < 128; ++k) {
          const double t = arow[k] * e4m3fn_to_f64(b_q[n * K + kb * 128 + k]);
          p += t;
          pabs += fabs(t);
        }
        acc += (double)s * p;
        accabs += fabs((double)s) * pabs;
      }
      c[m * N + n] = acc;
      cabs[m * N + n] = accabs;
    }
  }
  return 0;
}
