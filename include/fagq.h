/*
 * fagq.h - C ABI of the MI355X (gfx950) fused residual-add + RMSNorm +
 * per-token-group quantization operator.
 *
 * Reference interface replaced (paths relative to the reference repository
 * sinpeyw/flagos-kernelgen-72h-shanghai-2026):
 *   src/task01_fused_add_rmsnorm_group_quant.py:1731-1741
 *     fused_add_rmsnorm_group_quant(x, residual, gamma, residual_out,
 *                                   norm_out, x_q, x_scale, eps, group_size)
 *   and the kernels it routes to on a ROCm device:
 *     :1127-1348 (+ :1066-1124)  _preweighted_segmented_streaming_kernel (M >= 128)
 *     :65-121                    _preweighted_full_row_kernel (M < 128, via :1548-1728)
 *
 * The reference is a Python function over torch tensors; this library is the
 * native boundary under that function.  Every pointer is a device pointer,
 * every tensor is contiguous row-major unless the argument says otherwise,
 * and every call is stream-ordered: nothing here synchronizes the host,
 * allocates device memory, or throws.
 *
 * Numerics (per row of D elements, groups of G consecutive elements):
 *   r        = fp32(x) + fp32(residual)              (fp32, unrounded)
 *   residual_out = bf16_rne(r)
 *   sumsq    = sum r^2, accumulated in fp64, rounded once to fp32
 *   inv_rms  = fp32( 1 / sqrt( fp32(sumsq / D) + eps ) )  (correctly rounded)
 *   w        = r * fp32(gamma)
 *   norm     = w * inv_rms                           (norm_out = bf16_rne(norm))
 *   s_g      = max( max_{j in g}|w_j| * (inv_rms / QMAX), 1e-12 )
 *   F32 scales:   scale_g = s_g,   t = norm * (1 / s_g)
 *   UE8M0 scales: e_g = ceil(log2(s_g)) (exact, from the fp32 bits),
 *                 scale byte = e_g + 127,  t = ldexp(norm, -e_g)
 *   q        = encode(clamp(t, -QMAX, QMAX))
 *     FP8_E4M3FN: OCP e4m3fn, round-to-nearest-even, QMAX = 448
 *     INT8 + RNE: round half to even, QMAX = 127
 *     INT8 + TRUNC: round toward zero, QMAX = 127 (what the reference's
 *                   float->int cast does, task01.py:112-116 and :1100-1104)
 */
#ifndef FAGQ_H
#define FAGQ_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FAGQ_API __attribute__((visibility("default")))

/* Quantized-code formats (the dtype of x_q). */
enum fagq_q_format {
  FAGQ_Q_INT8 = 0,        /* int8, QMAX 127 (the reference's x_q dtype) */
  FAGQ_Q_FP8_E4M3FN = 1   /* OCP fp8 e4m3fn, QMAX 448 */
};

/* Scale formats (the dtype of x_scale). */
enum fagq_scale_format {
  FAGQ_SCALE_F32 = 0,     /* fp32 scale per group (the reference's x_scale dtype) */
  FAGQ_SCALE_UE8M0 = 1    /* uint8 biased exponent: scale = 2^(byte - 127) */
};

/* Scale layouts.  Logical shape is [M, D/G] in both cases. */
enum fagq_scale_layout {
  FAGQ_LAYOUT_ROW_MAJOR = 0,  /* scale[m * (D/G) + g]  (reference: task01.py:121) */
  FAGQ_LAYOUT_COL_MAJOR = 1   /* scale[g * M + m]     (physical [D/G, M]) */
};

/* Rounding of int8 codes.  fp8 codes always round to nearest even. */
enum fagq_rounding {
  FAGQ_ROUND_RNE = 0,
  FAGQ_ROUND_TRUNC = 1        /* reference-compatible int8 truncation */
};

/* Status codes.  0 = success, > 0 = argument rejected before any device
 * work, < 0 = -(hipError_t) reported by the HIP runtime. */
enum fagq_status {
  FAGQ_OK = 0,
  FAGQ_E_NULL = 1,          /* a required pointer is NULL */
  FAGQ_E_SHAPE = 2,         /* M < 0, D <= 0 or D % group_size != 0 (so D % 64 == 0) */
  FAGQ_E_GROUP = 3,         /* group_size not in {64, 128, 256} */
  FAGQ_E_ALIGN = 4,         /* a pointer is not aligned as required */
  FAGQ_E_FORMAT = 5,        /* unknown enum value or unsupported combination */
  FAGQ_E_EPS = 6,           /* eps negative or not finite */
  FAGQ_E_TOO_LARGE = 7,     /* D > FAGQ_MAX_D, M > INT32_MAX, or column-major scales
                               past 2^32 - 16 bytes */
  FAGQ_E_DEVICE = 8,        /* current device is not gfx950 */
  FAGQ_E_ALIAS = 9          /* an output overlaps an input it must not overlap */
};

#define FAGQ_MAX_D 32768

/*
 * fagq_launch - the fused operator (replaces task01.py:1731-1851).
 *
 *   x, residual      bf16 [M, D], 16-byte aligned
 *   gamma            bf16 [D], 16-byte aligned
 *   residual_out     bf16 [M, D], 16-byte aligned; may be the same pointer
 *                    as residual (in-place residual update); must not
 *                    partially overlap x or residual
 *   norm_out         bf16 [M, D], 16-byte aligned, or NULL (3-output form)
 *   q                int8 or fp8 [M, D], 8-byte aligned
 *   scale            fp32 (4-byte aligned) or uint8 per scale_format,
 *                    laid out per scale_layout
 *   M >= 0 rows (M == 0 is a no-op), D > 0 with D % group_size == 0,
 *   D <= FAGQ_MAX_D, group_size in {64, 128, 256}, eps >= 0 and finite.
 *   stream           hipStream_t (NULL = the legacy default stream)
 *
 * Every row is produced by exactly one workgroup; no atomics, no scratch.
 */
FAGQ_API int fagq_launch(const void* x, const void* residual, const void* gamma,
                         void* residual_out, void* norm_out, void* q, void* scale,
                         int64_t M, int64_t D, int64_t group_size, float eps,
                         int q_format, int scale_format, int scale_layout,
                         int rounding, void* stream);

/* Element types of the typed form. */
enum fagq_dtype { FAGQ_DT_BF16 = 0, FAGQ_DT_F16 = 1, FAGQ_DT_F32 = 2 };

/*
 * fagq_launch_typed - fagq_launch for other element types, as the reference
 * accepts them: its kernels convert every load to fp32 (task01.py:88-89,
 * :93-94) and every store to the destination's type (:91, :118), so fp16
 * activations or an fp32 residual stream run through the same operator
 * (src/task01_fused_add_rmsnorm_group_quant.py:1731-1741).
 *
 *   act_dtype        element type of x, gamma and norm_out
 *   res_dtype        element type of residual and residual_out
 *   (act_dtype, res_dtype) in {(BF16, BF16) (= fagq_launch), (F16, F16),
 *   (BF16, F32), (F16, F32), (F32, F32)}; other pairs FAGQ_E_FORMAT.
 *
 * Loads convert to fp32 exactly; residual_out and norm_out are rounded to
 * their type to nearest even (fp16 overflows to +-inf).  From r = x +
 * residual on, the definition is fagq_launch's.  Every x / residual /
 * gamma / residual_out / norm_out pointer is 16-byte aligned; residual_out
 * may be exactly residual (or x when both have the same element type).
 * Other arguments, limits and statuses as for fagq_launch.
 */
FAGQ_API int fagq_launch_typed(const void* x, const void* residual, const void* gamma,
                               void* residual_out, void* norm_out, void* q, void* scale,
                               int64_t M, int64_t D, int64_t group_size, float eps,
                               int q_format, int scale_format, int scale_layout, int rounding,
                               int act_dtype, int res_dtype, void* stream);

/* Multi-input form: the epilogue of a tensor-parallel reduction.  x is the
 * sum of nparts partial tensors (one per rank of a row-parallel layer, e.g.
 * the contributions a reduce-scatter gathers for this rank's rows), added in
 * fp32 in index order before the residual:
 *
 *   r = ((x_parts[0] + x_parts[1]) + ... + x_parts[nparts - 1]) + residual
 *
 * and everything after r is fagq_launch's definition.  The sum is never
 * rounded to bf16.  With nparts == 1 the outputs equal
 * fagq_launch(x_parts[0], ...) bit for bit.
 *
 * No counterpart in the reference: its operator takes one x
 * (src/task01_fused_add_rmsnorm_group_quant.py:1731-1741).  This is the
 * producer side of the path for tensor-parallel layers.
 *
 *   x_parts          host array of nparts device pointers, each bf16 [M, D],
 *                    16-byte aligned; 1 <= nparts <= FAGQ_MAX_PARTS
 *   residual_out     may be exactly residual; must not overlap any part
 *   3-output form (no norm_out); D <= FAGQ_MAX_D_PARTS; other arguments as
 *   for fagq_launch.
 */
#define FAGQ_MAX_PARTS 8
#define FAGQ_MAX_D_PARTS 16384

FAGQ_API int fagq_launch_parts(const void* const* x_parts, int nparts, const void* residual,
                               const void* gamma, void* residual_out, void* q, void* scale,
                               int64_t M, int64_t D, int64_t group_size, float eps,
                               int q_format, int scale_format, int scale_layout, int rounding,
                               void* stream);

/* Route description chosen by fagq_launch for a shape and scale format (for
 * tests and the benchmark).  waves_per_row * steps_per_wave * 512 >= D. */
typedef struct fagq_route {
  int32_t waves_per_row;    /* waves that split one row (1 = wave-per-row) */
  int32_t steps_per_wave;   /* 512-column steps each wave keeps in VGPRs */
  int32_t rows_per_block;   /* rows (row groups of waves_per_row waves) per workgroup */
  int32_t row_group_mode;   /* 0: independent rows; 1: gamma loaded once per workgroup and
                               shared through LDS; 2: as 1, and the column-major scales of
                               the workgroup's rows stored together */
  int32_t block_threads;    /* workgroup size */
  int32_t lds_bytes;        /* dynamic LDS reserved per workgroup (0: none) */
  int64_t grid_blocks;      /* workgroups launched */
  int32_t xcd_remap;        /* workgroup -> row order (see fagq_launch_mapped) */
  int32_t reserved;         /* zero */
} fagq_route;

/* Same validation as fagq_launch for the shape arguments; fills *route.
 * Never touches the device. */
FAGQ_API int fagq_query_route(int64_t M, int64_t D, int64_t group_size, int scale_format,
                              int scale_layout, fagq_route* route);

/* The route fagq_launch_parts takes for nparts partials (1..FAGQ_MAX_PARTS) of a
 * shape: independent rows (row_group_mode 0), 4 steps per wave for 6 or more
 * partials at 12..16 steps of 512 columns, else 2 (or FAGQ_PARTS_STEPS = 1).
 * The same shape checks as fagq_launch_parts (D <= FAGQ_MAX_D_PARTS); never
 * touches the device. */
FAGQ_API int fagq_query_route_parts(int64_t M, int64_t D, int64_t group_size, int nparts,
                                    int scale_format, int scale_layout, fagq_route* route);

/* The route fagq_launch_typed takes for an element-type pair: fagq_launch's
 * for (BF16, BF16) and (F16, F16); for the pairs with an fp32 tensor, the
 * typed kernel's (independent rows, row_group_mode 0).  Other pairs
 * FAGQ_E_FORMAT.  Never touches the device. */
FAGQ_API int fagq_query_route_typed(int64_t M, int64_t D, int64_t group_size, int scale_format,
                                    int scale_layout, int act_dtype, int res_dtype,
                                    fagq_route* route);

/* Static description of a status code; never NULL. */
FAGQ_API const char* fagq_status_string(int status);

/* Library ABI version (major * 10000 + minor * 100 + patch). */
FAGQ_API int fagq_version(void);

#ifdef __cplusplus
}
#endif

#endif /* FAGQ_H */
