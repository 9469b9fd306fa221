// fagq_api.hip - C ABI of the fused residual-add + RMSNorm + group-quant
// operator: argument validation, the route table, the per-device gfx950
// check, and launches on the caller's stream.
//
// Replaces the reference's Python entry and routers
// (src/task01_fused_add_rmsnorm_group_quant.py:1731-1851 and :1548-1728) and
// its per-call backend tagging (:13-62): the route is a pure function of
// (M, D), the device check is done once per device, and nothing here
// allocates, synchronizes or throws.
#include <atomic>
#include <cmath>
#include <cstdlib>
#include <cstring>

#include "fagq.h"
#include "fagq_diag.h"
#include "fagq_dispatch.hpp"

namespace fagq {
namespace {

// Plain 16-byte-vector copy, for calibrating HBM byte counters.
__global__ void __launch_bounds__(256) fagq_copy16(const u32x4* __restrict__ src,
                                                   u32x4* __restrict__ dst, int64_t n16) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += stride)
    __builtin_nontemporal_store(__builtin_nontemporal_load(src + i), dst + i);
}

constexpr int kVersion = 1 * 10000 + 0 * 100 + 0;
constexpr int kMaxDevices = 64;

struct Mapping {
  int wpr;        // waves per row
  int ns;         // steps per wave
  int rpb;        // row groups per workgroup
  int rseq;       // rows each row group processes in turn
  int block;      // threads per workgroup
  int64_t grid;   // workgroups
};

// Route-table knobs, read once: FAGQ_PREFILL_ROWS is the row count from which
// rows are split into 2-step waves (FAGQ_PREFILL_STEPS) instead of 1-step
// waves; FAGQ_PREFILL_RSEQ sets the rows each row group processes in turn
// (1 by default: prefetching a second row measured no faster).
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

int prefill_rseq() {
  static const int v = env_int("FAGQ_PREFILL_RSEQ", 1);
  return v;
}

// Workgroup -> row-tile order (see tile_of_block): column-major scales put
// neighbouring rows' scale words next to each other, so chunks of 8 (fp32)
// or 32 (ue8m0) consecutive row tiles go to one XCD and leave its L2 as full
// 32-byte writes; otherwise dispatch order.  FAGQ_XCD_REMAP overrides.
int remap_for(int scale_layout, int scale_format, int rpb) {
  static const int forced = [] {
    const char* s = std::getenv("FAGQ_XCD_REMAP");
    return s ? std::atoi(s) : -1;
  }();
  if (forced >= 0) return forced;
  if (scale_layout != FAGQ_LAYOUT_COL_MAJOR) return 0;
  const int rows = scale_format == FAGQ_SCALE_F32 ? 8 : 32;
  return rows / rpb > 1 ? rows / rpb : 0;
}

bool valid_remap(int r) { return r == 0 || r == 1 || (r >= 2 && r <= 64 && (r & (r - 1)) == 0); }

int ceil_div(int64_t a, int64_t b) { return (int)((a + b - 1) / b); }

// Completes a mapping from (wpr, rpb, rseq); returns false if it is not launchable.
bool finish_mapping(int64_t M, int D, int wpr, int rpb, int rseq, Mapping* m) {
  const int steps = ceil_div(D, kStepCols);
  if (wpr < 1 || wpr > kMaxWavesPerBlock || rpb < 1 || wpr * rpb > kMaxWavesPerBlock) return false;
  if (rseq_index(rseq) < 0) return false;
  const int ns = ceil_div(steps, wpr);
  if (ns > kMaxStepsPerWave) return false;
  m->wpr = wpr;
  m->ns = ns;
  m->rpb = rpb;
  m->rseq = rseq;
  m->block = 64 * wpr * rpb;
  const int64_t per_block = (int64_t)rpb * rseq;
  m->grid = (M + per_block - 1) / per_block;
  return m->grid <= INT32_MAX;
}

// The route table.  Each row is split over waves of one workgroup so that
// every wave streams only 1-2 KB of each input per step (dispatch-ordered
// workgroups then keep the set of rows in flight small, which HBM rewards).
// Prefill (M >= prefill_rows()): 2 steps per wave, one row per workgroup.
// Decode: 1 step per wave, one row per workgroup, as many waves as the row
// has steps (<= 16).
// Rows of more than 16 steps use up to 4 steps per wave.
void choose_mapping(int64_t M, int D, Mapping* m) {
  const int steps = ceil_div(D, kStepCols);
  const bool prefill = M >= prefill_rows();
  int ns = prefill ? prefill_steps() : 1;
  if (ns > kMaxStepsPerWave) ns = kMaxStepsPerWave;
  const int min_ns = ceil_div(steps, kMaxWavesPerBlock);
  if (ns < min_ns) ns = min_ns;
  if (ns > steps) ns = steps;
  const int wpr = ceil_div(steps, ns);
  const int rpb = wpr >= 4 ? 1 : 4 / wpr;
  int rseq = prefill ? prefill_rseq() : 1;
  if (rseq_index(rseq) < 0) rseq = 1;
  finish_mapping(M, D, wpr, rpb, rseq, m);
}

bool aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }

struct Range {
  uintptr_t lo, hi;
};

bool overlap(Range a, Range b) { return a.lo < b.hi && b.lo < a.hi; }

int validate(const void* x, const void* residual, const void* gamma, const void* residual_out,
             const void* norm_out, const void* q, const void* scale, int64_t M, int64_t D,
             int64_t G, float eps, int q_format, int scale_format, int scale_layout,
             int rounding) {
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
  // Column-major scales are addressed with 32-bit buffer offsets.
  if (scale_layout == FAGQ_LAYOUT_COL_MAJOR &&
      M * (D / G) * (scale_format == FAGQ_SCALE_F32 ? 4 : 1) > (int64_t)UINT32_MAX)
    return FAGQ_E_TOO_LARGE;
  if (!(eps >= 0.0f) || !std::isfinite(eps)) return FAGQ_E_EPS;
  if (!aligned(x, 16) || !aligned(residual, 16) || !aligned(gamma, 16) ||
      !aligned(residual_out, 16) || (norm_out && !aligned(norm_out, 16)) || !aligned(q, 8) ||
      (scale_format == FAGQ_SCALE_F32 && !aligned(scale, 4)))
    return FAGQ_E_ALIGN;
  if (M == 0) return FAGQ_OK;

  // Byte ranges.  residual_out may be exactly x or residual (each element is
  // read by the lane that later writes it); everything else is disjoint.
  const uintptr_t nb = (uintptr_t)(M * D * 2);
  const uintptr_t sb = (uintptr_t)(M * (D / G) * (scale_format == FAGQ_SCALE_F32 ? 4 : 1));
  auto rng = [](const void* p, uintptr_t n) {
    return Range{reinterpret_cast<uintptr_t>(p), reinterpret_cast<uintptr_t>(p) + n};
  };
  const Range in[3] = {rng(x, nb), rng(residual, nb), rng(gamma, (uintptr_t)D * 2)};
  const Range ro = rng(residual_out, nb), qo = rng(q, nb / 2), so = rng(scale, sb);
  const Range no = norm_out ? rng(norm_out, nb) : Range{0, 0};
  for (int i = 0; i < 3; ++i) {
    const bool exact_ok = (i < 2) && ro.lo == in[i].lo;
    if (overlap(ro, in[i]) && !exact_ok) return FAGQ_E_ALIAS;
    if (overlap(qo, in[i]) || overlap(so, in[i]) || (norm_out && overlap(no, in[i])))
      return FAGQ_E_ALIAS;
  }
  if (overlap(ro, qo) || overlap(ro, so) || overlap(qo, so)) return FAGQ_E_ALIAS;
  if (norm_out && (overlap(no, ro) || overlap(no, qo) || overlap(no, so))) return FAGQ_E_ALIAS;
  return FAGQ_OK;
}

}  // namespace

// gfx950 check, done once per device.
int device_check() {
  static std::atomic<int> cache[kMaxDevices];   // 0 unknown, 1 gfx950, 2 other
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return -(int)e;
  if (dev < 0 || dev >= kMaxDevices) return FAGQ_E_DEVICE;
  int c = cache[dev].load(std::memory_order_relaxed);
  if (c == 0) {
    hipDeviceProp_t prop;
    e = hipGetDeviceProperties(&prop, dev);
    if (e != hipSuccess) return -(int)e;
    c = std::strncmp(prop.gcnArchName, "gfx950", 6) == 0 ? 1 : 2;
    cache[dev].store(c, std::memory_order_relaxed);
  }
  return c == 1 ? FAGQ_OK : FAGQ_E_DEVICE;
}

namespace {

LaunchFn lookup(int q_format, int scale_format, int rounding, int lpg_idx, int steps, bool norm,
                int rseq) {
  const int qf = q_format == FAGQ_Q_FP8_E4M3FN ? QF_FP8
                 : rounding == FAGQ_ROUND_RNE  ? QF_I8_RNE
                                               : QF_I8_TRUNC;
  const bool ue = scale_format == FAGQ_SCALE_UE8M0;
  const int ri = rseq_index(rseq);
  switch (qf) {
    case QF_FP8:
      return ue ? lookup_q0_s1(lpg_idx, steps, norm, ri) : lookup_q0_s0(lpg_idx, steps, norm, ri);
    case QF_I8_RNE:
      return ue ? lookup_q1_s1(lpg_idx, steps, norm, ri) : lookup_q1_s0(lpg_idx, steps, norm, ri);
    default:
      return ue ? lookup_q2_s1(lpg_idx, steps, norm, ri) : lookup_q2_s0(lpg_idx, steps, norm, ri);
  }
}

LaunchFn lookup_parts(int q_format, int scale_format, int rounding, int lpg_idx, int steps) {
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

// The multi-input form's mapping: FAGQ_PARTS_STEPS (default 2; 1 measured
// 5 % slower at D = 7168) steps per wave, 2 whenever the row would need more
// than 16 waves; one row per row group; small rows share a workgroup as in
// choose_mapping.
void choose_mapping_parts(int64_t M, int D, Mapping* m) {
  const int steps = ceil_div(D, kStepCols);
  int ns = parts_steps() >= kMaxStepsParts ? kMaxStepsParts : 1;
  if (ceil_div(steps, ns) > kMaxWavesPerBlock) ns = kMaxStepsParts;
  if (ns > steps) ns = steps;
  const int wpr = ceil_div(steps, ns);
  const int rpb = wpr >= 4 ? 1 : 4 / wpr;
  finish_mapping(M, D, wpr, rpb, 1, m);
}

void fill_args(KArgs* a, const Mapping& m, const void* x, const void* residual, const void* gamma,
               void* residual_out, void* norm_out, void* q, void* scale, int64_t M, int64_t D,
               int64_t G, float eps, int scale_layout, int remap) {
  a->x = static_cast<const uint16_t*>(x);
  a->res = static_cast<const uint16_t*>(residual);
  a->gamma = static_cast<const uint16_t*>(gamma);
  a->res_out = static_cast<uint16_t*>(residual_out);
  a->norm_out = static_cast<uint16_t*>(norm_out);
  a->q = static_cast<uint8_t*>(q);
  a->scale = static_cast<uint8_t*>(scale);
  a->M = M;
  a->D = (int32_t)D;
  a->groups = (int32_t)(D / G);
  a->eps = eps;
  a->wpr = m.wpr;
  a->rpb = m.rpb;
  a->col_major = scale_layout == FAGQ_LAYOUT_COL_MAJOR;
  a->remap = remap;
  a->remap_shift = remap >= 2 ? __builtin_ctz((unsigned)remap) : 0;
  a->wpr_magic = (65536 + m.wpr - 1) / m.wpr;
  a->nparts = 0;
  for (int p = 0; p < kMaxParts; ++p) a->xparts[p] = nullptr;
}

int launch_with(const Mapping& m, const void* x, const void* residual, const void* gamma,
                void* residual_out, void* norm_out, void* q, void* scale, int64_t M, int64_t D,
                int64_t G, float eps, int q_format, int scale_format, int scale_layout,
                int rounding, int remap, void* stream) {
  const int dc = device_check();
  if (dc != FAGQ_OK) return dc;
  KArgs a;
  fill_args(&a, m, x, residual, gamma, residual_out, norm_out, q, scale, M, D, G, eps,
            scale_layout, remap);
  const LaunchFn fn = lookup(q_format, scale_format, rounding, lpg_index((int)G), m.ns,
                             norm_out != nullptr, m.rseq);
  const hipError_t e = fn(a, dim3((unsigned)m.grid), dim3((unsigned)m.block),
                          static_cast<hipStream_t>(stream));
  return e == hipSuccess ? FAGQ_OK : -(int)e;
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
  choose_mapping(M, (int)D, &m);
  return launch_with(m, x, residual, gamma, residual_out, norm_out, q, scale, M, D, group_size,
                     eps, q_format, scale_format, scale_layout, rounding,
                     remap_for(scale_layout, scale_format, m.rpb * m.rseq), stream);
}

FAGQ_API int fagq_launch_mapped(const void* x, const void* residual, const void* gamma,
                                void* residual_out, void* norm_out, void* q, void* scale,
                                int64_t M, int64_t D, int64_t group_size, float eps,
                                int q_format, int scale_format, int scale_layout, int rounding,
                                int waves_per_row, int rows_per_block, int rows_in_sequence,
                                int xcd_remap, void* stream) {
  const int v = validate(x, residual, gamma, residual_out, norm_out, q, scale, M, D, group_size,
                         eps, q_format, scale_format, scale_layout, rounding);
  if (v != FAGQ_OK) return v;
  Mapping m;
  if (!finish_mapping(M, (int)D, waves_per_row, rows_per_block, rows_in_sequence, &m))
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
  choose_mapping_parts(M, (int)D, &m);
  KArgs a;
  fill_args(&a, m, x_parts[0], residual, gamma, residual_out, nullptr, q, scale, M, D, group_size,
            eps, scale_layout, remap_for(scale_layout, scale_format, m.rpb));
  a.nparts = nparts;
  for (int p = 0; p < nparts; ++p) a.xparts[p] = static_cast<const uint16_t*>(x_parts[p]);
  const LaunchFn fn = lookup_parts(q_format, scale_format, rounding, lpg_index((int)group_size), m.ns);
  const hipError_t e = fn(a, dim3((unsigned)m.grid), dim3((unsigned)m.block),
                          static_cast<hipStream_t>(stream));
  return e == hipSuccess ? FAGQ_OK : -(int)e;
}

FAGQ_API int fagq_query_route(int64_t M, int64_t D, int64_t group_size, fagq_route* route) {
  if (!route) return FAGQ_E_NULL;
  if (group_size != 64 && group_size != 128 && group_size != 256) return FAGQ_E_GROUP;
  if (M < 0 || D <= 0 || D % group_size != 0) return FAGQ_E_SHAPE;
  if (D > FAGQ_MAX_D || M > (int64_t)INT32_MAX) return FAGQ_E_TOO_LARGE;
  Mapping m;
  choose_mapping(M, (int)D, &m);
  route->waves_per_row = m.wpr;
  route->steps_per_wave = m.ns;
  route->rows_per_block = m.rpb;
  route->rows_in_sequence = m.rseq;
  route->block_threads = m.block;
  route->reserved = 0;
  route->grid_blocks = m.grid;
  return FAGQ_OK;
}

FAGQ_API int fagq_diag_encode(const float* in, void* out, int64_t n, int q_format, int rounding,
                              void* stream) {
  if (!in || !out) return FAGQ_E_NULL;
  if (n < 0 || n % 8 != 0) return FAGQ_E_SHAPE;
  if (!aligned(in, 16) || !aligned(out, 8)) return FAGQ_E_ALIGN;
  if (q_format != FAGQ_Q_INT8 && q_format != FAGQ_Q_FP8_E4M3FN) return FAGQ_E_FORMAT;
  if (rounding != FAGQ_ROUND_RNE && rounding != FAGQ_ROUND_TRUNC) return FAGQ_E_FORMAT;
  if (q_format == FAGQ_Q_FP8_E4M3FN && rounding != FAGQ_ROUND_RNE) return FAGQ_E_FORMAT;
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
  const void* k = q_format == FAGQ_Q_FP8_E4M3FN ? reinterpret_cast<const void*>(&fagq_encode<QF_FP8>)
                  : rounding == FAGQ_ROUND_RNE ? reinterpret_cast<const void*>(&fagq_encode<QF_I8_RNE>)
                                               : reinterpret_cast<const void*>(&fagq_encode<QF_I8_TRUNC>);
  const hipError_t e = hipLaunchKernel(k, grid, block, args, 0, s);
  return e == hipSuccess ? FAGQ_OK : -(int)e;
}

FAGQ_API int fagq_diag_copy(const void* src, void* dst, int64_t bytes, void* stream) {
  if (!src || !dst) return FAGQ_E_NULL;
  if (bytes < 0 || bytes % 16 != 0) return FAGQ_E_SHAPE;
  if (!aligned(src, 16) || !aligned(dst, 16)) return FAGQ_E_ALIGN;
  if (bytes == 0) return FAGQ_OK;
  const int dc = device_check();
  if (dc != FAGQ_OK) return dc;
  const int64_t n16 = bytes / 16;
  const int64_t want = (n16 + 255) / 256;
  const dim3 grid((unsigned)(want < 8192 ? want : 8192)), block(256);
  const u32x4* s4 = static_cast<const u32x4*>(src);
  u32x4* d4 = static_cast<u32x4*>(dst);
  int64_t count16 = n16;
  void* args[] = {&s4, &d4, &count16};
  const hipError_t e = hipLaunchKernel(reinterpret_cast<const void*>(&fagq_copy16), grid, block,
                                       args, 0, static_cast<hipStream_t>(stream));
  return e == hipSuccess ? FAGQ_OK : -(int)e;
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
