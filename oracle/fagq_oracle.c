/*
 * fagq_oracle.c - CPU restatement of the reference's fused residual-add +
 * RMSNorm + per-token-group quantization, used ONLY as the checker by the
 * tests, by __graft_entry__.smoke() and by bench.py's cpu_baseline leg.  It
 * is test infrastructure: the product path (the HIP library) never links,
 * loads or calls it.
 *
 * Reference algorithm (sinpeyw/flagos-kernelgen-72h-shanghai-2026,
 * src/task01_fused_add_rmsnorm_group_quant.py), the AMD route:
 *   r = fp32(x) + fp32(residual)                    :88-89, :1151-1157
 *   residual_out = bf16(r)                          :91, :1160
 *   sumsq = sum r^2 ; inv = rsqrt(sumsq / D + eps)  :90, :100, :1274-1278
 *   w = r * fp32(gamma)  ("preweighted")            :93-94, :1163-1164
 *   gmax = max |w| over each group                  :95-98, :1165-1167
 *   norm = w * inv                                  :101, :1089
 *   scale = max(gmax * (inv / QMAX), 1e-12)         :102, :1090
 *   q = cast(clamp(norm * (1 / scale), -QMAX, QMAX)):103-116, :1091-1104
 * The reference's reduction order (tl.sum) and tl.rsqrt are compiler- and
 * hardware-defined; this restatement evaluates them exactly rounded:
 * sumsq accumulated in fp64 (each r^2 is exact there) and rounded once to
 * fp32, inv = fp32(1 / sqrt(double(v))).  The GPU library evaluates the
 * same definition.  Formats beyond the reference (fp8 e4m3fn, int8
 * round-half-even, ue8m0 scales, column-major scales) follow the same
 * formulas with QMAX = 448 for fp8.
 *
 * Build: gcc -O2 -std=c11 -fPIC -shared -fopenmp -ffp-contract=off (see
 * oracle/build.py).  Floating point must be IEEE single/double with
 * round-to-nearest-even and no contraction, which is x86-64 SSE code.
 */
#include <math.h>
#include <omp.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define ORC_API __attribute__((visibility("default")))

static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

static inline float bf16_to_f32(uint16_t b) { return u2f((uint32_t)b << 16); }

/* fp32 -> bf16, round to nearest even; NaN stays NaN (quiet). */
static inline uint16_t f32_to_bf16(float f) {
  uint32_t u = f2u(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x0040u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

/* IEEE binary16 -> fp32, exactly (subnormals, infinities, NaN payloads). */
static inline float f16_to_f32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  const uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
  if (e == 0) {                                    /* zero or subnormal: m * 2^-24 */
    const float v = ldexpf((float)m, -24);
    return sign ? -v : v;
  }
  if (e == 31) return u2f(sign | 0x7f800000u | (m << 13));
  return u2f(sign | ((e + 112u) << 23) | (m << 13));
}

/* fp32 -> IEEE binary16, round to nearest even: |v| >= 65520 (the tie above
 * the largest finite 65504) becomes +-inf; below 2^-14 the result is the
 * subnormal rint(|v| * 2^24) * 2^-24 (1024 there is 2^-14, the smallest
 * normal); NaN stays NaN (quiet). */
static inline uint16_t f32_to_f16(float f) {
  const uint32_t u = f2u(f);
  const uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
  const uint32_t a = u & 0x7fffffffu;
  if (a > 0x7f800000u) return (uint16_t)(sign | 0x7e00u | ((a >> 13) & 0x3ffu));
  if (a >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);
  if (a < 0x38800000u) return (uint16_t)(sign | (uint16_t)rintf(u2f(a) * 16777216.0f));
  /* rebias the exponent (127 -> 15) and round the 23-bit mantissa to 10 bits */
  return (uint16_t)(sign | ((a - 0x38000000u + 0x0fffu + ((a >> 13) & 1u)) >> 13));
}

/* fp32 -> OCP fp8 e4m3fn (bias 7, 3 mantissa bits, no infinities, max 448,
 * S.1111.111 = NaN), round to nearest even.  |v| >= 464 rounds past 448 and
 * gives NaN (no saturation), as a plain IEEE-style conversion does. */
static inline uint8_t f32_to_e4m3fn(float v) {
  const uint8_t sign = (uint8_t)((f2u(v) >> 24) & 0x80u);
  if (isnan(v)) return (uint8_t)(sign | 0x7fu);
  const float a = fabsf(v);
  if (a == 0.0f) return sign;
  int e2;
  (void)frexpf(a, &e2);           /* a = m * 2^e2, m in [0.5, 1) */
  int E = e2 - 1;                 /* a in [2^E, 2^(E+1)) */
  if (E > 8) return (uint8_t)(sign | 0x7fu);
  const int p = (E < -6 ? -6 : E) - 3;      /* spacing 2^p of the target binade */
  const float n = rintf(ldexpf(a, -p));      /* exact scaling, then RNE */
  if (n == 0.0f) return sign;
  /* value = n * 2^p; renormalise (n may have rounded up to 16). */
  int ni = (int)n;
  int pe = p;
  while (ni >= 16) { ni >>= 1; pe += 1; }   /* ni even when it reaches 16 */
  if (ni < 8) return (uint8_t)(sign | ni);  /* subnormal: 2^-9 * ni (pe == -9) */
  const int exp_field = pe + 3 + 7;         /* value = (ni/8) * 2^(pe+3) */
  if (exp_field > 15 || (exp_field == 15 && (ni - 8) == 7)) return (uint8_t)(sign | 0x7fu);
  return (uint8_t)(sign | (exp_field << 3) | (ni - 8));
}

/* ceil(log2(s)) for a positive normal fp32 s, from the bits. */
static inline int ceil_log2_bits(float s) {
  const uint32_t b = f2u(s);
  return (int)(b >> 23) - 127 + ((b & 0x7fffffu) != 0u);
}

enum { Q_INT8 = 0, Q_FP8 = 1 };
enum { S_F32 = 0, S_UE8M0 = 1 };
enum { L_ROW = 0, L_COL = 1 };
enum { R_RNE = 0, R_TRUNC = 1 };

static inline uint8_t encode(float t, int q_format, int rounding) {
  if (q_format == Q_FP8) return f32_to_e4m3fn(t);
  const float v = rounding == R_RNE ? rintf(t) : t;
  return (uint8_t)(int8_t)(int)v;   /* C conversion truncates toward zero */
}

/* ---- element-wise entry points (vectorised over arrays) ---- */

ORC_API void orc_bf16_from_f32(const float* in, uint16_t* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = f32_to_bf16(in[i]);
}

ORC_API void orc_f16_from_f32(const float* in, uint16_t* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = f32_to_f16(in[i]);
}

ORC_API void orc_f32_from_f16(const uint16_t* in, float* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = f16_to_f32(in[i]);
}

/* Codes for already-scaled values, after the operator's clamp. */
ORC_API void orc_encode(const float* in, uint8_t* out, int64_t n, int q_format, int rounding) {
  const float qmax = q_format == Q_FP8 ? 448.0f : 127.0f;
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < n; ++i) {
    const float t = fminf(fmaxf(in[i], -qmax), qmax);
    out[i] = encode(t, q_format, rounding);
  }
}

/* Raw e4m3fn conversion without the clamp (for checking against casts). */
ORC_API void orc_e4m3fn_raw(const float* in, uint8_t* out, int64_t n) {
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < n; ++i) out[i] = f32_to_e4m3fn(in[i]);
}

ORC_API void orc_ceil_log2(const float* in, int32_t* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = ceil_log2_bits(in[i]);
}

/* ---- the operator ---- */

/*
 * Same argument meaning as fagq_launch_parts (include/fagq.h), host pointers:
 * x is the sum of nparts partial tensors x_parts[0..nparts-1], added in fp32
 * in index order, r = ((x_0 + x_1) + ... + x_{P-1}) + residual.  With one part
 * this is the operator's r = fp32(x) + fp32(residual) (task01.py:88-89).
 * norm_out may be NULL.  nthreads <= 0 uses the OpenMP default.
 * Returns 0, or 1 on an argument this restatement does not accept.
 */
ORC_API int orc_fagq_parts(const uint16_t* const* x_parts, int nparts, const uint16_t* residual,
                           const uint16_t* gamma, uint16_t* residual_out, uint16_t* norm_out,
                           uint8_t* q, void* scale, int64_t M, int64_t D, int64_t G, float eps,
                           int q_format, int scale_format, int scale_layout, int rounding,
                           int nthreads) {
  if (nparts < 1 || nparts > 8) return 1;
  if (M < 0 || D <= 0 || G <= 0 || D % G != 0) return 1;
  if (q_format == Q_FP8 && rounding != R_RNE) return 1;
  const float qmax = q_format == Q_FP8 ? 448.0f : 127.0f;
  const int64_t groups = D / G;
  int ok = 0;
#pragma omp parallel num_threads(nthreads > 0 ? nthreads : omp_get_max_threads()) if (M > 1)
  {
    float* w = (float*)malloc((size_t)D * sizeof(float));
    if (!w) {
#pragma omp atomic write
      ok = 1;
    } else {
#pragma omp for schedule(static)
      for (int64_t m = 0; m < M; ++m) {
        const uint16_t* rr = residual + m * D;
        uint16_t* ro = residual_out + m * D;
        double ss = 0.0;
        for (int64_t j = 0; j < D; ++j) {
          float xs = bf16_to_f32(x_parts[0][m * D + j]);
          for (int p = 1; p < nparts; ++p) xs = xs + bf16_to_f32(x_parts[p][m * D + j]);
          const float r = xs + bf16_to_f32(rr[j]);
          ro[j] = f32_to_bf16(r);
          ss += (double)r * (double)r;
          w[j] = r * bf16_to_f32(gamma[j]);
        }
        const float sumsq = (float)ss;
        const float mean = sumsq / (float)D;
        const float inv = (float)(1.0 / sqrt((double)(mean + eps)));
        const float inv_q = inv / qmax;
        for (int64_t g = 0; g < groups; ++g) {
          float gmax = 0.0f;
          for (int64_t j = g * G; j < (g + 1) * G; ++j) gmax = fmaxf(gmax, fabsf(w[j]));
          const float s = fmaxf(gmax * inv_q, 1.0e-12f);
          const int64_t si = scale_layout == L_COL ? g * M + m : m * groups + g;
          float mul = 0.0f;
          int e = 0;
          if (scale_format == S_F32) {
            mul = 1.0f / s;
            ((float*)scale)[si] = s;
          } else {
            e = ceil_log2_bits(s);
            if (e > 127) e = 127;
            ((uint8_t*)scale)[si] = (uint8_t)(e + 127);
          }
          for (int64_t j = g * G; j < (g + 1) * G; ++j) {
            const float n = w[j] * inv;
            if (norm_out) norm_out[m * D + j] = f32_to_bf16(n);
            const float u = scale_format == S_F32 ? n * mul : ldexpf(n, -e);
            const float t = fminf(fmaxf(u, -qmax), qmax);
            q[m * D + j] = encode(t, q_format, rounding);
          }
        }
      }
      free(w);
    }
  }
  return ok;
}

/* The operator (task01.py:1731-1741 semantics): one x tensor. */
ORC_API int orc_fagq(const uint16_t* x, const uint16_t* residual, const uint16_t* gamma,
                     uint16_t* residual_out, uint16_t* norm_out, uint8_t* q, void* scale,
                     int64_t M, int64_t D, int64_t G, float eps, int q_format,
                     int scale_format, int scale_layout, int rounding, int nthreads) {
  const uint16_t* parts[1] = {x};
  return orc_fagq_parts(parts, 1, residual, gamma, residual_out, norm_out, q, scale, M, D, G,
                        eps, q_format, scale_format, scale_layout, rounding, nthreads);
}

/* ---- the typed form (fagq_launch_typed, include/fagq.h) ---- */

enum { DT_BF16 = 0, DT_F16 = 1, DT_F32 = 2 };

static inline float load_elem(const void* p, int64_t i, int dt) {
  if (dt == DT_F32) return ((const float*)p)[i];
  const uint16_t h = ((const uint16_t*)p)[i];
  return dt == DT_F16 ? f16_to_f32(h) : bf16_to_f32(h);
}

static inline void store_elem(void* p, int64_t i, int dt, float v) {
  if (dt == DT_F32) ((float*)p)[i] = v;
  else ((uint16_t*)p)[i] = dt == DT_F16 ? f32_to_f16(v) : f32_to_bf16(v);
}

/*
 * The operator with x, gamma and norm_out of element type act_dtype and
 * residual, residual_out of res_dtype (DT_BF16, DT_F16 or DT_F32): every
 * load is converted to fp32 and every store rounded to its type, as the
 * reference's kernels do (task01.py:88-89, :93-94, :91, :118); the
 * arithmetic is orc_fagq_parts' with one part.  Host pointers; norm_out may
 * be NULL.  Returns 0, or 1 on an argument this restatement does not accept.
 */
ORC_API int orc_fagq_typed(const void* x, const void* residual, const void* gamma,
                           void* residual_out, void* norm_out, uint8_t* q, void* scale,
                           int64_t M, int64_t D, int64_t G, float eps, int q_format,
                           int scale_format, int scale_layout, int rounding, int act_dtype,
                           int res_dtype, int nthreads) {
  if (M < 0 || D <= 0 || G <= 0 || D % G != 0) return 1;
  if (q_format == Q_FP8 && rounding != R_RNE) return 1;
  if (act_dtype < DT_BF16 || act_dtype > DT_F32 || res_dtype < DT_BF16 || res_dtype > DT_F32)
    return 1;
  const float qmax = q_format == Q_FP8 ? 448.0f : 127.0f;
  const int64_t groups = D / G;
  int ok = 0;
#pragma omp parallel num_threads(nthreads > 0 ? nthreads : omp_get_max_threads()) if (M > 1)
  {
    float* w = (float*)malloc((size_t)D * sizeof(float));
    if (!w) {
#pragma omp atomic write
      ok = 1;
    } else {
#pragma omp for schedule(static)
      for (int64_t m = 0; m < M; ++m) {
        double ss = 0.0;
        for (int64_t j = 0; j < D; ++j) {
          const int64_t i = m * D + j;
          const float r = load_elem(x, i, act_dtype) + load_elem(residual, i, res_dtype);
          store_elem(residual_out, i, res_dtype, r);
          ss += (double)r * (double)r;
          w[j] = r * load_elem(gamma, j, act_dtype);
        }
        const float sumsq = (float)ss;
        const float mean = sumsq / (float)D;
        const float inv = (float)(1.0 / sqrt((double)(mean + eps)));
        const float inv_q = inv / qmax;
        for (int64_t g = 0; g < groups; ++g) {
          float gmax = 0.0f;
          for (int64_t j = g * G; j < (g + 1) * G; ++j) gmax = fmaxf(gmax, fabsf(w[j]));
          const float s = fmaxf(gmax * inv_q, 1.0e-12f);
          const int64_t si = scale_layout == L_COL ? g * M + m : m * groups + g;
          float mul = 0.0f;
          int e = 0;
          if (scale_format == S_F32) {
            mul = 1.0f / s;
            ((float*)scale)[si] = s;
          } else {
            e = ceil_log2_bits(s);
            if (e > 127) e = 127;
            ((uint8_t*)scale)[si] = (uint8_t)(e + 127);
          }
          for (int64_t j = g * G; j < (g + 1) * G; ++j) {
            const float n = w[j] * inv;
            if (norm_out) store_elem(norm_out, m * D + j, act_dtype, n);
            const float u = scale_format == S_F32 ? n * mul : ldexpf(n, -e);
            const float t = fminf(fmaxf(u, -qmax), qmax);
            q[m * D + j] = encode(t, q_format, rounding);
          }
        }
      }
      free(w);
    }
  }
  return ok;
}
