// fagq_api.hip - C ABI of the fused residual-add + RMSNorm + group-quant
// operator: argument validation, the route table and launches on the
// caller's stream (the per-device gfx950 check is fagq_device.hip's).
//
// Replaces the reference's Python entry and routers
// (src/task01_fused_add_rmsnorm_group_quant.py:1731-1851 and :1548-1728) and
// its per-call backend tagging (:13-62): the route is a pure function of
// (M, D), the device check is done once per device, and nothing here
// allocates, synchronizes or throws.
#include <cmath>
#include <cstdlib>
#include <cstring>

#include "fagq.h"
#include "fagq_diag.h"
#include "fagq_dispatch.hpp"

namespace fagq {
namespace {

constexpr int kVersion = 1 * 10000 + 0 * 100 + 0;

struct Mapping {
  int wpr;        // waves per row
  int ns;         // steps per wave
  int rpb;        // row groups (rows) per workgroup
  int mode;       // RowGroupMode
  int block;      // threads per workgroup
  int lds;        // dynamic LDS bytes reserved per workgroup (caps workgroups per CU)
  int64_t grid;   // workgroups
};

constexpr int kMaxDynLds = 65536;

// Route-table knobs, read once: FAGQ_PREFILL_ROWS is the row count from which
// rows are split into 2-step waves (FAGQ_PREFILL_STEPS) instead of 1-step
// waves.
int env_int(const char* name, int dflt) {
  const char* s = std::getenv(name);
  const int v = s ? std::atoi(s) : 0;
  return v > 0 ? v : dflt;
}

int prefill_rows() {
  static const int v = env_int("FAGQ_PREFILL_ROWS", 1024);
  return v;
}

int prefill_steps() {
  static const int v = env_int("FAGQ_PREFILL_STEPS", 2);
  return v;
}

// Workgroup -> row-tile order (see tile_of_block): column-major scales put
// neighbouring rows' scale words next to each other, so chunks of 8 (fp32)
// or 32 (ue8m0) consecutive rows go to one XCD and leave its L2 as full
// 32-byte writes (16 fp32 rows when a workgroup stores two rows' words at
// once, measured best at 16384 x 7168); otherwise dispatch order.
// FAGQ_XCD_REMAP overrides with any valid remap (0, 1 or a power of two up
// to 64); other values are ignored.
bool valid_remap(int r) { return r == 0 || r == 1 || (r >= 2 && r <= 64 && (r & (r - 1)) == 0); }

int remap_for(int scale_layout, int scale_format, int rpb, int mode) {
  static const int forced = [] {
    const char* s = std::getenv("FAGQ_XCD_REMAP");
    const int v = s ? std::atoi(s) : -1;
    return valid_remap(v) ? v : -1;
  }();
  if (forced >= 0) return forced;
  if (scale_layout != FAGQ_LAYOUT_COL_MAJOR) return 0;
  const int rows = scale_format == FAGQ_SCALE_F32 ? (mode == RG_WIDE_SCALES ? 16 : 8) : 32;
  return rows / rpb > 1 ? rows / rpb : 0;
}

int ceil_div(int64_t a, int64_t b) { return (int)((a + b - 1) / b); }

// Completes a mapping from (wpr, rpb, mode, lds); returns false if it is not
// launchable.  The shared modes need the row's steps to fit the LDS gamma
// buffer (wpr * ns <= 16, i.e. D <= 8192); the wide-scale mode stores 2 or 4
// rows' words at once.
bool finish_mapping(int64_t M, int D, int wpr, int rpb, int mode, int lds, Mapping* m) {
  const int steps = ceil_div(D, kStepCols);
  if (wpr < 1 || wpr > kMaxWavesPerBlock || rpb < 1 || wpr * rpb > kMaxWavesPerBlock) return false;
  if (mode < 0 || mode >= kNumModes || lds < 0 || lds > kMaxDynLds) return false;
  const int ns = ceil_div(steps, wpr);
  if (ns > kMaxStepsPerWave) return false;
  if (mode != RG_INDEPENDENT && wpr * ns > kMaxSharedSteps) return false;
  if (mode == RG_WIDE_SCALES && rpb != 2 && rpb != kMaxWideRows) return false;
  m->wpr = wpr;
  m->ns = ns;
  m->rpb = rpb;
  m->mode = mode;
  m->block = 64 * wpr * rpb;
  m->lds = lds;
  m->grid = (M + rpb - 1) / rpb;
  return m->grid <= INT32_MAX;
}

// The route table.  Each row is split over waves of one workgroup so that
// every wave streams only 1-4 KB of each input (dispatch-ordered workgroups
// then keep the set of rows in flight small, which HBM rewards).  Rows below
// refer to prefill (M >= prefill_rows()) unless stated; timings are medians of
// interleaved runs at M = 16384 (MI355X):
// * column-major scales, 12..16 steps (5632 < D <= 8192): two rows per
//   workgroup of 4-step waves, gamma loaded once and shared through LDS, each
//   group's scale words of both rows stored together (RG_WIDE_SCALES).
//   D = 7168 fp32: 130.2 us against 134.6 us for one row of 2-step waves;
//   D = 7168 ue8m0: 130.8 against 134.2; D = 8192 fp32: 147.0 against 151.0.
// * row-major, 12..14 steps: one row of 2-step waves, at most three
//   workgroups per CU (48 KB of LDS reserved each): D = 7168: 130.3 against
//   132.5 us; D = 6144: 112.2 against 113.5.
// * row-major, 15..16 steps: two rows of 4-step waves sharing gamma
//   (RG_SHARED_GAMMA): D = 8192: 149.3 against 150.5 us.
// * 5..8 steps: 1-step waves: D = 4096: 21.3 against 21.6 us at M = 4096,
//   74.7 against 75.5 at M = 16384; D = 3072: 57.5 against 59.0.
// * 9..11 steps: 2-step waves, one row per workgroup, at most four
//   workgroups per CU (36 KB of LDS reserved each): D = 5120, M = 16384:
//   94.4 against 95.8 us (ue8m0 column-major), 94.8 against 96.2 (fp32
//   column-major), 93.4 against 94.7 (fp32 row-major); M = 8192 ue8m0:
//   49.2 against 49.8; D = 4608: 85.4 against 86.7; D = 5632: 104.8 against
//   105.7.  Three per CU was slower than either (D = 4608: 88.2).
// * other prefill: 2 steps per wave, one row per workgroup.
// * decode: 1 step per wave, one row per workgroup, as many waves as the row
//   has steps (<= 16).
// Rows of more than 16 steps use up to 4 steps per wave.
// Rows split into waves of 1 step (decode, and prefill rows of 5..8 steps)
// or FAGQ_PREFILL_STEPS steps, independent row groups: the route for every
// shape the cases of choose_mapping below leave, and for the typed form.
void default_mapping(int64_t M, int D, Mapping* m) {
  const int steps = ceil_div(D, kStepCols);
  const bool prefill = M >= prefill_rows();
  int ns = prefill ? (steps >= 5 && steps <= 8 ? 1 : prefill_steps()) : 1;
  if (ns > kMaxStepsPerWave) ns = kMaxStepsPerWave;
  const int min_ns = ceil_div(steps, kMaxWavesPerBlock);
  if (ns < min_ns) ns = min_ns;
  if (ns > steps) ns = steps;
  const int wpr = ceil_div(steps, ns);
  const int rpb = wpr >= 4 ? 1 : 4 / wpr;
  // 36 KB per workgroup: four fit in the CU's 160 KB of LDS with the static
  // arrays, five do not.
  const int lds = prefill && ns == 2 && rpb == 1 && steps >= 9 && steps <= 11 ? 36 * 1024 : 0;
  finish_mapping(M, D, wpr, rpb, RG_INDEPENDENT, lds, m);
}

void choose_mapping(int64_t M, int D, int scale_format, int scale_layout, Mapping* m) {
  const int steps = ceil_div(D, kStepCols);
  const bool prefill = M >= prefill_rows();
  const bool col = scale_layout == FAGQ_LAYOUT_COL_MAJOR;
  (void)scale_format;
  if (prefill && steps >= 12 && steps <= kMaxSharedSteps) {
    const int wpr4 = ceil_div(steps, kMaxStepsPerWave);
    if (col && finish_mapping(M, D, wpr4, 2, RG_WIDE_SCALES, 0, m)) return;
    if (!col && steps >= 15 && finish_mapping(M, D, wpr4, 2, RG_SHARED_GAMMA, 0, m)) return;
    if (!col && finish_mapping(M, D, ceil_div(steps, 2), 1, RG_INDEPENDENT, 48 * 1024, m)) return;
  }
  default_mapping(M, D, m);
}

bool aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }

struct Range {
  uintptr_t lo, hi;
};

bool overlap(Range a, Range b) { return a.lo < b.hi && b.lo < a.hi; }

// Argument checks of the operator; ba and br are the element sizes of the
// activation tensors (x, gamma, norm_out) and of the residual stream
// (residual, residual_out): 2 for bf16 / fp16, 4 for fp32.
int validate(const void* x, const void* residual, const void* gamma, const void* residual_out,
             const void* norm_out, const void* q, const void* scale, int64_t M, int64_t D,
             int64_t G, float eps, int q_format, int scale_format, int scale_layout,
             int rounding, uintptr_t ba = 2, uintptr_t br = 2) {
  if (!x || !residual || !gamma || !residual_out || !q || !scale) return FAGQ_E_NULL;
  if (q_format != FAGQ_Q_INT8 && q_format != FAGQ_Q_FP8_E4M3FN) return FAGQ_E_FORMAT;
  if (scale_format != FAGQ_SCALE_F32 && scale_format != FAGQ_SCALE_UE8M0) return FAGQ_E_FORMAT;
  if (scale_layout != FAGQ_LAYOUT_ROW_MAJOR && scale_layout != FAGQ_LAYOUT_COL_MAJOR)
    return FAGQ_E_FORMAT;
  if (rounding != FAGQ_ROUND_RNE && rounding != FAGQ_ROUND_TRUNC) return FAGQ_E_FORMAT;
  if (q_format == FAGQ_Q_FP8_E4M3FN && rounding != FAGQ_ROUND_RNE) return FAGQ_E_FORMAT;
  if (G != 64 && G != 128 && G != 256) return FAGQ_E_GROUP;
  if (M < 0 || D <= 0 || D % G != 0) return FAGQ_E_SHAPE;
  if (D > FAGQ_MAX_D || M > (int64_t)INT32_MAX) return FAGQ_E_TOO_LARGE;
  // Column-major scales are addressed with 32-bit buffer offsets, and lanes
  // without a group store at offset 0xffffffff, which must stay outside.
  if (scale_layout == FAGQ_LAYOUT_COL_MAJOR &&
      M * (D / G) * (scale_format == FAGQ_SCALE_F32 ? 4 : 1) > (int64_t)UINT32_MAX - 16)
    return FAGQ_E_TOO_LARGE;
  if (!(eps >= 0.0f) || !std::isfinite(eps)) return FAGQ_E_EPS;
  if (!aligned(x, 16) || !aligned(residual, 16) || !aligned(gamma, 16) ||
      !aligned(residual_out, 16) || (norm_out && !aligned(norm_out, 16)) || !aligned(q, 8) ||
      (scale_format == FAGQ_SCALE_F32 && !aligned(scale, 4)))
    return FAGQ_E_ALIGN;
  if (M == 0) return FAGQ_OK;

  // Byte ranges.  residual_out may be exactly residual, or x when x has the
  // residual stream's element type (each element is read by the lane that
  // later writes it); everything else is disjoint.
  const uintptr_t ne = (uintptr_t)(M * D);
  const uintptr_t sb = (uintptr_t)(M * (D / G) * (scale_format == FAGQ_SCALE_F32 ? 4 : 1));
  auto rng = [](const void* p, uintptr_t n) {
    return Range{reinterpret_cast<uintptr_t>(p), reinterpret_cast<uintptr_t>(p) + n};
  };
  const Range in[3] = {rng(x, ne * ba), rng(residual, ne * br), rng(gamma, (uintptr_t)D * ba)};
  const Range ro = rng(residual_out, ne * br), qo = rng(q, ne), so = rng(scale, sb);
  const Range no = norm_out ? rng(norm_out, ne * ba) : Range{0, 0};
  for (int i = 0; i < 3; ++i) {
    const bool exact_ok = ((i == 0 && ba == br) || i == 1) && ro.lo == in[i].lo;
    if (overlap(ro, in[i]) && !exact_ok) return FAGQ_E_ALIAS;
    if (overlap(qo, in[i]) || overlap(so, in[i]) || (norm_out && overlap(no, in[i])))
      return FAGQ_E_ALIAS;
  }
  if (overlap(ro, qo) || overlap(ro, so) || overlap(qo, so)) return FAGQ_E_ALIAS;
  if (norm_out && (overlap(no, ro) || overlap(no, qo) || overlap(no, so))) return FAGQ_E_ALIAS;
  return FAGQ_OK;
}

// fagq_rows for bf16 tensors, or (f16) for the typed form's fp16 tensors.
LaunchFn lookup(int q_format, int scale_format, int rounding, int lpg_idx, int steps, bool norm,
                int mode, bool f16 = false) {
  const int qf = q_format == FAGQ_Q_FP8_E4M3FN ? QF_FP8
                 : rounding == FAGQ_ROUND_RNE  ? QF_I8_RNE
                                               : QF_I8_TRUNC;
  const bool ue = scale_format == FAGQ_SCALE_UE8M0;
  const int ri = mode;
  if (f16) {
    switch (qf) {
      case QF_FP8:
        return ue ? lookup_f16_q0_s1(lpg_idx, steps, norm, ri)
                  : lookup_f16_q0_s0(lpg_idx, steps, norm, ri);
      case QF_I8_RNE:
        return ue ? lookup_f16_q1_s1(lpg_idx, steps, norm, ri)
                  : lookup_f16_q1_s0(lpg_idx, steps, norm, ri);
      default:
        return ue ? lookup_f16_q2_s1(lpg_idx, steps, norm, ri)
                  : lookup_f16_q2_s0(lpg_idx, steps, norm, ri);
    }
  }
  switch (qf) {
    case QF_FP8:
      return ue ? lookup_q0_s1(lpg_idx, steps, norm, ri) : lookup_q0_s0(lpg_idx, steps, norm, ri);
    case QF_I8_RNE:
      return ue ? lookup_q1_s1(lpg_idx, steps, norm, ri) : lookup_q1_s0(lpg_idx, steps, norm, ri);
    default:
      return ue ? lookup_q2_s1(lpg_idx, steps, norm, ri) : lookup_q2_s0(lpg_idx, steps, norm, ri);
  }
}

// fagq_rows_typed, family in [TF_BF16_R32, TF_F32] (fp16 tensors alone run fagq_rows).
LaunchFn lookup_typed(int q_format, int scale_format, int rounding, int lpg_idx, int steps,
                      bool norm, int family) {
  const int qf = q_format == FAGQ_Q_FP8_E4M3FN ? QF_FP8
                 : rounding == FAGQ_ROUND_RNE  ? QF_I8_RNE
                                               : QF_I8_TRUNC;
  const bool ue = scale_format == FAGQ_SCALE_UE8M0;
  switch (qf) {
    case QF_FP8:
      return ue ? lookup_typed_q0_s1(lpg_idx, steps, norm, family)
                : lookup_typed_q0_s0(lpg_idx, steps, norm, family);
    case QF_I8_RNE:
      return ue ? lookup_typed_q1_s1(lpg_idx, steps, norm, family)
                : lookup_typed_q1_s0(lpg_idx, steps, norm, family);
    default:
      return ue ? lookup_typed_q2_s1(lpg_idx, steps, norm, family)
                : lookup_typed_q2_s0(lpg_idx, steps, norm, family);
  }
}

// Type family of an (activation, residual-stream) element-type pair; -1 if
// the pair is not supported (or is the bf16 pair, which fagq_launch serves).
int type_family(int act_dtype, int res_dtype) {
  if (act_dtype == FAGQ_DT_F16 && res_dtype == FAGQ_DT_F16) return TF_F16;
  if (act_dtype == FAGQ_DT_BF16 && res_dtype == FAGQ_DT_F32) return TF_BF16_R32;
  if (act_dtype == FAGQ_DT_F16 && res_dtype == FAGQ_DT_F32) return TF_F16_R32;
  if (act_dtype == FAGQ_DT_F32 && res_dtype == FAGQ_DT_F32) return TF_F32;
  return -1;
}

PartsLaunchFn lookup_parts(int q_format, int scale_format, int rounding, int lpg_idx, int steps) {
  const int qf = q_format == FAGQ_Q_FP8_E4M3FN ? QF_FP8
                 : rounding == FAGQ_ROUND_RNE  ? QF_I8_RNE
                                               : QF_I8_TRUNC;
  const bool ue = scale_format == FAGQ_SCALE_UE8M0;
  switch (qf) {
    case QF_FP8: return ue ? lookup_parts_q0_s1(lpg_idx, steps) : lookup_parts_q0_s0(lpg_idx, steps);
    case QF_I8_RNE: return ue ? lookup_parts_q1_s1(lpg_idx, steps) : lookup_parts_q1_s0(lpg_idx, steps);
    default: return ue ? lookup_parts_q2_s1(lpg_idx, steps) : lookup_parts_q2_s0(lpg_idx, steps);
  }
}

int parts_steps() {
  static const int v = env_int("FAGQ_PARTS_STEPS", 2);
  return v;
}

// The multi-input form's mapping, one row per row group (small rows share a
// workgroup as in choose_mapping):
// * at least 6 partials and 12..16 steps (5632 < D <= 8192): 4-step waves,
//   each holding 4 KB of every partial in flight, 2 waves per SIMD.  Medians
//   of interleaved runs at D = 7168, against 2-step waves: 2048 rows with 8
//   partials 51.7 against 52.9 us, with 6 partials 41.9 against 42.6; 4096
//   rows with 8 partials 100.5 against 102.6; 1024 rows 27.2 against 27.7.
//   With 4 partials even (61.6 against 61.8 us at 4096 rows), with 2 or 1
//   slower (88.5 against 84.7 at 8192 rows, 139.4 against 137.0 at 16384);
//   3-step waves (5 per row, 3 waves per SIMD) slower everywhere (60.7 us
//   at 2048 rows with 8 partials).
// * otherwise FAGQ_PARTS_STEPS (default 2; 1 measured 5 % slower at D =
//   7168) steps per wave, 2 whenever the row would need more than 16 waves.
void choose_mapping_parts(int64_t M, int D, int nparts, Mapping* m) {
  const int steps = ceil_div(D, kStepCols);
  int ns;
  if (nparts >= 6 && steps >= 12 && steps <= 16) {
    ns = 4;
  } else {
    ns = parts_steps() >= 2 ? 2 : 1;
    if (ceil_div(steps, ns) > kMaxWavesPerBlock) ns = 2;
    if (ns > steps) ns = steps;
  }
  const int wpr = ceil_div(steps, ns);
  const int rpb = wpr >= 4 ? 1 : 4 / wpr;
  finish_mapping(M, D, wpr, rpb, RG_INDEPENDENT, 0, m);
}

void fill_args(KArgs* a, const Mapping& m, const void* x, const void* residual, const void* gamma,
               void* residual_out, void* norm_out, void* q, void* scale, int64_t M, int64_t D,
               int64_t G, float eps, int scale_format, int scale_layout, int remap) {
  a->x = static_cast<const uint16_t*>(x);
  a->res = static_cast<const uint16_t*>(residual);
  a->gamma = static_cast<const uint16_t*>(gamma);
  a->res_out = static_cast<uint16_t*>(residual_out);
  a->norm_out = static_cast<uint16_t*>(norm_out);
  a->q = static_cast<uint8_t*>(q);
  a->scale = static_cast<uint8_t*>(scale);
  a->M = (int32_t)M;
  a->D = (int32_t)D;
  a->groups = (int32_t)(D / G);
  a->eps = eps;
  const uintptr_t wide_bytes =
      (uintptr_t)m.rpb * (uintptr_t)(scale_format == FAGQ_SCALE_F32 ? 4 : 1);
  const int wide_ok = m.mode == RG_WIDE_SCALES && M % m.rpb == 0 &&
                      (reinterpret_cast<uintptr_t>(scale) % wide_bytes) == 0;
  a->cfg = KArgs::pack_cfg(m.wpr, m.rpb, remap, remap >= 2 ? __builtin_ctz((unsigned)remap) : 0,
                           scale_layout == FAGQ_LAYOUT_COL_MAJOR, wide_ok);
  a->wpr_magic = (65536 + m.wpr - 1) / m.wpr;
}

int launch_with(const Mapping& m, const void* x, const void* residual, const void* gamma,
                void* residual_out, void* norm_out, void* q, void* scale, int64_t M, int64_t D,
                int64_t G, float eps, int q_format, int scale_format, int scale_layout,
                int rounding, int remap, void* stream, bool f16 = false) {
  const int dc = device_check();
  if (dc != FAGQ_OK) return dc;
  KArgs a;
  fill_args(&a, m, x, residual, gamma, residual_out, norm_out, q, scale, M, D, G, eps,
            scale_format, scale_layout, remap);
  const LaunchFn fn = lookup(q_format, scale_format, rounding, lpg_index((int)G), m.ns,
                             norm_out != nullptr, m.mode, f16);
  return fn(a, dim3((unsigned)m.grid), dim3((unsigned)m.block), (unsigned)m.lds,
            static_cast<hipStream_t>(stream));
}

// Shape checks shared by the route queries (those of validate() that need no
// pointers).
int check_route_shape(int64_t M, int64_t D, int64_t group_size, int scale_format,
                      int scale_layout, const fagq_route* route) {
  if (!route) return FAGQ_E_NULL;
  if (group_size != 64 && group_size != 128 && group_size != 256) return FAGQ_E_GROUP;
  if (M < 0 || D <= 0 || D % group_size != 0) return FAGQ_E_SHAPE;
  if (D > FAGQ_MAX_D || M > (int64_t)INT32_MAX) return FAGQ_E_TOO_LARGE;
  if (scale_format != FAGQ_SCALE_F32 && scale_format != FAGQ_SCALE_UE8M0) return FAGQ_E_FORMAT;
  if (scale_layout != FAGQ_LAYOUT_ROW_MAJOR && scale_layout != FAGQ_LAYOUT_COL_MAJOR)
    return FAGQ_E_FORMAT;
  return FAGQ_OK;
}

void fill_route(const Mapping& m, int scale_format, int scale_layout, fagq_route* route) {
  route->waves_per_row = m.wpr;
  route->steps_per_wave = m.ns;
  route->rows_per_block = m.rpb;
  route->row_group_mode = m.mode;
  route->block_threads = m.block;
  route->lds_bytes = m.lds;
  route->grid_blocks = m.grid;
  route->xcd_remap = remap_for(scale_layout, scale_format, m.rpb, m.mode);
  route->reserved = 0;
}

}  // namespace
}  // namespace fagq

using namespace fagq;

extern "C" {

FAGQ_API int fagq_launch(const void* x, const void* residual, const void* gamma,
                         void* residual_out, void* norm_out, void* q, void* scale, int64_t M,
                         int64_t D, int64_t group_size, float eps, int q_format,
                         int scale_format, int scale_layout, int rounding, void* stream) {
  const int v = validate(x, residual, gamma, residual_out, norm_out, q, scale, M, D, group_size,
                         eps, q_format, scale_format, scale_layout, rounding);
  if (v != FAGQ_OK || M == 0) return v;
  Mapping m;
  choose_mapping(M, (int)D, scale_format, scale_layout, &m);
  return launch_with(m, x, residual, gamma, residual_out, norm_out, q, scale, M, D, group_size,
                     eps, q_format, scale_format, scale_layout, rounding,
                     remap_for(scale_layout, scale_format, m.rpb, m.mode), stream);
}

FAGQ_API int fagq_launch_typed(const void* x, const void* residual, const void* gamma,
                               void* residual_out, void* norm_out, void* q, void* scale,
                               int64_t M, int64_t D, int64_t group_size, float eps,
                               int q_format, int scale_format, int scale_layout, int rounding,
                               int act_dtype, int res_dtype, void* stream) {
  if (act_dtype == FAGQ_DT_BF16 && res_dtype == FAGQ_DT_BF16)
    return fagq_launch(x, residual, gamma, residual_out, norm_out, q, scale, M, D, group_size, eps,
                       q_format, scale_format, scale_layout, rounding, stream);
  const int tf = type_family(act_dtype, res_dtype);
  if (tf < 0) return FAGQ_E_FORMAT;
  if (tf == TF_F16) {
    // fp16 tensors: the bf16 operator's kernels and route, with fp16 elements.
    const int v = validate(x, residual, gamma, residual_out, norm_out, q, scale, M, D, group_size,
                           eps, q_format, scale_format, scale_layout, rounding);
    if (v != FAGQ_OK || M == 0) return v;
    Mapping m;
    choose_mapping(M, (int)D, scale_format, scale_layout, &m);
    return launch_with(m, x, residual, gamma, residual_out, norm_out, q, scale, M, D, group_size,
                       eps, q_format, scale_format, scale_layout, rounding,
                       remap_for(scale_layout, scale_format, m.rpb, m.mode), stream, true);
  }
  const uintptr_t ba = act_dtype == FAGQ_DT_F32 ? 4 : 2, br = res_dtype == FAGQ_DT_F32 ? 4 : 2;
  const int v = validate(x, residual, gamma, residual_out, norm_out, q, scale, M, D, group_size,
                         eps, q_format, scale_format, scale_layout, rounding, ba, br);
  if (v != FAGQ_OK || M == 0) return v;
  const int dc = device_check();
  if (dc != FAGQ_OK) return dc;
  Mapping m;
  default_mapping(M, (int)D, &m);
  KArgs a;
  fill_args(&a, m, x, residual, gamma, residual_out, norm_out, q, scale, M, D, group_size, eps,
            scale_format, scale_layout, remap_for(scale_layout, scale_format, m.rpb, m.mode));
  const LaunchFn fn = lookup_typed(q_format, scale_format, rounding, lpg_index((int)group_size),
                                   m.ns, norm_out != nullptr, tf);
  return fn(a, dim3((unsigned)m.grid), dim3((unsigned)m.block), (unsigned)m.lds,
            static_cast<hipStream_t>(stream));
}

FAGQ_API int fagq_launch_mapped(const void* x, const void* residual, const void* gamma,
                                void* residual_out, void* norm_out, void* q, void* scale,
                                int64_t M, int64_t D, int64_t group_size, float eps,
                                int q_format, int scale_format, int scale_layout, int rounding,
                                int waves_per_row, int rows_per_block, int row_group_mode,
                                int xcd_remap, int lds_bytes, void* stream) {
  const int v = validate(x, residual, gamma, residual_out, norm_out, q, scale, M, D, group_size,
                         eps, q_format, scale_format, scale_layout, rounding);
  if (v != FAGQ_OK) return v;
  Mapping m;
  if (!finish_mapping(M, (int)D, waves_per_row, rows_per_block, row_group_mode, lds_bytes, &m))
    return FAGQ_E_FORMAT;
  if (row_group_mode == RG_WIDE_SCALES && scale_layout != FAGQ_LAYOUT_COL_MAJOR)
    return FAGQ_E_FORMAT;
  if (!valid_remap(xcd_remap)) return FAGQ_E_FORMAT;
  if (M == 0) return FAGQ_OK;
  return launch_with(m, x, residual, gamma, residual_out, norm_out, q, scale, M, D, group_size,
                     eps, q_format, scale_format, scale_layout, rounding, xcd_remap, stream);
}

FAGQ_API int fagq_launch_parts(const void* const* x_parts, int nparts, const void* residual,
                               const void* gamma, void* residual_out, void* q, void* scale,
                               int64_t M, int64_t D, int64_t group_size, float eps,
                               int q_format, int scale_format, int scale_layout, int rounding,
                               void* stream) {
  if (!x_parts) return FAGQ_E_NULL;
  if (nparts < 1 || nparts > FAGQ_MAX_PARTS) return FAGQ_E_SHAPE;
  for (int p = 0; p < nparts; ++p)
    if (!x_parts[p]) return FAGQ_E_NULL;
  // Common checks with part 0 standing for x (residual_out == x is not
  // allowed here: it is checked below against every part).
  const int v = validate(x_parts[0], residual, gamma, residual_out, nullptr, q, scale, M, D,
                         group_size, eps, q_format, scale_format, scale_layout, rounding);
  if (v != FAGQ_OK) return v;
  if (D > FAGQ_MAX_D_PARTS) return FAGQ_E_TOO_LARGE;
  if (M == 0) return FAGQ_OK;
  const uintptr_t nb = (uintptr_t)(M * D * 2);
  const uintptr_t sbytes =
      (uintptr_t)(M * (D / group_size) * (scale_format == FAGQ_SCALE_F32 ? 4 : 1));
  auto rng = [](const void* p, uintptr_t n) {
    return Range{reinterpret_cast<uintptr_t>(p), reinterpret_cast<uintptr_t>(p) + n};
  };
  const Range ro = rng(residual_out, nb), qo = rng(q, nb / 2), so = rng(scale, sbytes);
  for (int p = 0; p < nparts; ++p) {
    if (!aligned(x_parts[p], 16)) return FAGQ_E_ALIGN;
    const Range xp = rng(x_parts[p], nb);
    if (overlap(xp, ro) || overlap(xp, qo) || overlap(xp, so)) return FAGQ_E_ALIAS;
  }
  const int dc = device_check();
  if (dc != FAGQ_OK) return dc;
  Mapping m;
  choose_mapping_parts(M, (int)D, nparts, &m);
  PArgs a;
  fill_args(&a.k, m, x_parts[0], residual, gamma, residual_out, nullptr, q, scale, M, D,
            group_size, eps, scale_format, scale_layout,
            remap_for(scale_layout, scale_format, m.rpb, m.mode));
  a.nparts = nparts;
  for (int p = 0; p < kMaxParts; ++p)
    a.xparts[p] = p < nparts ? static_cast<const uint16_t*>(x_parts[p]) : nullptr;
  const PartsLaunchFn fn =
      lookup_parts(q_format, scale_format, rounding, lpg_index((int)group_size), m.ns);
  return fn(a, dim3((unsigned)m.grid), dim3((unsigned)m.block), 0u,
            static_cast<hipStream_t>(stream));
}

FAGQ_API int fagq_query_route(int64_t M, int64_t D, int64_t group_size, int scale_format,
                               int scale_layout, fagq_route* route) {
  return fagq_query_route_typed(M, D, group_size, scale_format, scale_layout, FAGQ_DT_BF16,
                                FAGQ_DT_BF16, route);
}

FAGQ_API int fagq_query_route_parts(int64_t M, int64_t D, int64_t group_size, int nparts,
                                    int scale_format, int scale_layout, fagq_route* route) {
  const int v = check_route_shape(M, D, group_size, scale_format, scale_layout, route);
  if (v != FAGQ_OK) return v;
  if (nparts < 1 || nparts > FAGQ_MAX_PARTS) return FAGQ_E_SHAPE;
  if (D > FAGQ_MAX_D_PARTS) return FAGQ_E_TOO_LARGE;
  Mapping m;
  choose_mapping_parts(M, (int)D, nparts, &m);
  fill_route(m, scale_format, scale_layout, route);
  return FAGQ_OK;
}

FAGQ_API int fagq_query_route_typed(int64_t M, int64_t D, int64_t group_size, int scale_format,
                                    int scale_layout, int act_dtype, int res_dtype,
                                    fagq_route* route) {
  const int v = check_route_shape(M, D, group_size, scale_format, scale_layout, route);
  if (v != FAGQ_OK) return v;
  const bool bf16 = act_dtype == FAGQ_DT_BF16 && res_dtype == FAGQ_DT_BF16;
  const int tf = bf16 ? -1 : type_family(act_dtype, res_dtype);
  if (!bf16 && tf < 0) return FAGQ_E_FORMAT;
  // fagq_launch_typed: bf16 and fp16 tensors take the operator's route, the
  // families with an fp32 tensor the typed kernel's default mapping.
  Mapping m;
  if (bf16 || tf == TF_F16) choose_mapping(M, (int)D, scale_format, scale_layout, &m);
  else default_mapping(M, (int)D, &m);
  fill_route(m, scale_format, scale_layout, route);
  return FAGQ_OK;
}

FAGQ_API int fagq_diag_encode(const float* in, void* out, int64_t n, int q_format, int rounding,
                              int clamp, void* stream) {
  if (!in || !out) return FAGQ_E_NULL;
  if (n < 0 || n % 8 != 0) return FAGQ_E_SHAPE;
  if (!aligned(in, 16) || !aligned(out, 8)) return FAGQ_E_ALIGN;
  if (q_format != FAGQ_Q_INT8 && q_format != FAGQ_Q_FP8_E4M3FN) return FAGQ_E_FORMAT;
  if (rounding != FAGQ_ROUND_RNE && rounding != FAGQ_ROUND_TRUNC) return FAGQ_E_FORMAT;
  if (q_format == FAGQ_Q_FP8_E4M3FN && rounding != FAGQ_ROUND_RNE) return FAGQ_E_FORMAT;
  if (clamp != 0 && clamp != 1) return FAGQ_E_FORMAT;
  if (n == 0) return FAGQ_OK;
  const int dc = device_check();
  if (dc != FAGQ_OK) return dc;
  const int64_t n8 = n / 8;
  const dim3 grid((unsigned)((n8 + 255) / 256)), block(256);
  const hipStream_t s = static_cast<hipStream_t>(stream);
  const float* src = in;
  u32x2* o = static_cast<u32x2*>(out);
  int64_t count8 = n8;
  void* args[] = {&src, &o, &count8};
  const int qf = q_format == FAGQ_Q_FP8_E4M3FN ? QF_FP8
                 : rounding == FAGQ_ROUND_RNE  ? QF_I8_RNE
                                               : QF_I8_TRUNC;
  static const void* const kernels[3][2] = {
      {reinterpret_cast<const void*>(&fagq_encode<QF_FP8, false>),
       reinterpret_cast<const void*>(&fagq_encode<QF_FP8, true>)},
      {reinterpret_cast<const void*>(&fagq_encode<QF_I8_RNE, false>),
       reinterpret_cast<const void*>(&fagq_encode<QF_I8_RNE, true>)},
      {reinterpret_cast<const void*>(&fagq_encode<QF_I8_TRUNC, false>),
       reinterpret_cast<const void*>(&fagq_encode<QF_I8_TRUNC, true>)}};
  return launch_kernel(kernels[qf][clamp], grid, block, args, 0, s);
}

FAGQ_API int fagq_diag_scale_offsets(int64_t M, int64_t D, int64_t group_size, int scale_format,
                                     int scale_layout, int waves_per_row, int64_t row,
                                     int64_t* out, int64_t cap) {
  if (!out) return FAGQ_E_NULL;
  if (group_size != 64 && group_size != 128 && group_size != 256) return FAGQ_E_GROUP;
  if (M <= 0 || D <= 0 || D % group_size != 0) return FAGQ_E_SHAPE;
  if (D > FAGQ_MAX_D || M > (int64_t)INT32_MAX) return FAGQ_E_TOO_LARGE;
  if (scale_format != FAGQ_SCALE_F32 && scale_format != FAGQ_SCALE_UE8M0) return FAGQ_E_FORMAT;
  if (scale_layout != FAGQ_LAYOUT_ROW_MAJOR && scale_layout != FAGQ_LAYOUT_COL_MAJOR)
    return FAGQ_E_FORMAT;
  const uint32_t sb = scale_format == FAGQ_SCALE_F32 ? 4u : 1u;
  const int col = scale_layout == FAGQ_LAYOUT_COL_MAJOR;
  if (col && M * (D / group_size) * sb > (int64_t)UINT32_MAX - 16) return FAGQ_E_TOO_LARGE;
  if (row < 0 || row >= M) return FAGQ_E_SHAPE;
  Mapping m;
  if (!finish_mapping(M, (int)D, waves_per_row, 1, RG_INDEPENDENT, 0, &m)) return FAGQ_E_FORMAT;
  if (cap < (int64_t)m.wpr * m.ns * 64) return FAGQ_E_SHAPE;
  const int G = (int)group_size, lpg = G / 8;
  const uint32_t gps = (uint32_t)(kStepCols / G);
  for (int part = 0; part < m.wpr; ++part) {
    const int c0 = part * m.ns * kStepCols;
    const uint32_t cols = D > c0 ? (uint32_t)(D - c0) : 0u;
    const ScaleSpan sp = scale_span(M, (int32_t)(D / G), col, sb, row, true, c0 / G, cols != 0);
    for (int k = 0; k < m.ns; ++k)
      for (int lane = 0; lane < 64; ++lane) {
        const uint32_t off = scale_lane_offset((uint32_t)(lane / lpg), (uint32_t)k, gps,
                                               sp.ngroups, sp.gstride);
        // A store of sb bytes at `off` lands only if it fits the descriptor.
        const bool lands = (uint64_t)off + sb <= (uint64_t)sp.bytes;
        out[((int64_t)part * m.ns + k) * 64 + lane] =
            lands ? sp.base + (int64_t)(off / sb) : -1;
      }
  }
  return FAGQ_OK;
}

FAGQ_API const char* fagq_status_string(int status) {
  switch (status) {
    case FAGQ_OK: return "ok";
    case FAGQ_E_NULL: return "a required pointer is NULL";
    case FAGQ_E_SHAPE: return "invalid shape (M < 0, D <= 0 or D % group_size != 0)";
    case FAGQ_E_GROUP: return "group_size must be 64, 128 or 256";
    case FAGQ_E_ALIGN: return "a pointer is not aligned as required";
    case FAGQ_E_FORMAT: return "unknown or unsupported format, layout, rounding or mapping";
    case FAGQ_E_EPS: return "eps must be finite and >= 0";
    case FAGQ_E_TOO_LARGE: return "D exceeds FAGQ_MAX_D or M exceeds INT32_MAX";
    case FAGQ_E_DEVICE: return "current device is not gfx950";
    case FAGQ_E_ALIAS: return "an output overlaps an input or another output";
    default: return status < 0 ? "HIP runtime error" : "unknown status";
  }
}

FAGQ_API int fagq_version(void) { return kVersion; }

}  // extern "C"
