// fagq_kernels.hpp - gfx950 device code of the fused residual-add + RMSNorm +
// per-token-group quantization operator.
//
// Reference dataflow restated here (reference repo paths):
//   src/task01_fused_add_rmsnorm_group_quant.py:88-121    (full-row kernel)
//   src/task01_fused_add_rmsnorm_group_quant.py:1148-1348 (segmented streaming
//                                                           kernel, AMD route)
//   src/task01_fused_add_rmsnorm_group_quant.py:1066-1124 (segment store)
//
// Work mapping.  A "step" is 512 consecutive columns of one row: 64 lanes x 8
// bf16 per lane, read with one 16-byte load per lane per tensor.  With 8
// elements per lane, a group of G columns covers G/8 consecutive lanes (16
// lanes = one DPP row for G = 128), so a group maximum is a 3..5-step
// DPP/permlane reduction that never leaves the wave.
//
// A row is split over wpr waves of one workgroup, each owning NS <= 4
// consecutive steps and keeping r * gamma for them in VGPRs, so every input
// byte is read from HBM once and no intermediate is written.  Only the fp64
// partial sums of squares cross waves, through LDS.  A workgroup holds rpb
// row groups (one row each); in the shared modes row group 0 alone loads
// gamma and hands it to the others through LDS, and may store the
// column-major scales of all rpb rows with one wide store per group.
//
// Every buffer access passes its whole offset as the VGPR offset (constant
// parts fold into the instruction's immediate offset) and a zero scalar
// offset.  With a register scalar offset the compiler assumes that a store
// of more than 8 bytes has read its data VGPRs at once and lets the next
// VALU overwrite them immediately; on gfx950 that lost the last 4 lanes of
// each 16-lane row of residual_out, nondeterministically.
//
// Memory is accessed through buffer descriptors (raw buffers, gfx9 format):
// each wave's descriptor for a row starts at its first column and is sized
// to the rest of the row, so lanes past the end of the row read zeros and
// their stores are dropped by the hardware, and a row past M gets an empty
// descriptor.  The step code therefore has no lane-dependent branches around
// memory operations (which would also make the compiler wait for stores
// whenever it waits for a later load), and addressing is one VGPR offset per
// lane plus scalar offsets.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace fagq {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

enum QFormat { QF_FP8 = 0, QF_I8_RNE = 1, QF_I8_TRUNC = 2 };
enum SFormat { SF_F32 = 0, SF_UE8M0 = 1 };

constexpr int kStepCols = 512;      // columns per wave step (64 lanes x 8)
constexpr int kMaxWavesPerBlock = 16;
constexpr int kMaxStepsPerWave = 4;
constexpr int kMaxParts = 8;        // partial sums of x in the multi-input form
constexpr int kMaxStepsParts = 4;   // steps per wave in the multi-input form (1, 2 or 4)

// Row-group modes of a workgroup of rpb row groups x wpr waves.
enum RowGroupMode {
  RG_INDEPENDENT = 0,   // every wave loads its gamma slice, every row group stores its scales
  RG_SHARED_GAMMA = 1,  // row group 0 loads gamma and hands it to the others through LDS
  RG_WIDE_SCALES = 2,   // RG_SHARED_GAMMA, and row group 0 stores the column-major scales of
                        // the rpb consecutive rows of the workgroup with one store per group
};
constexpr int kNumModes = 3;
constexpr int kMaxSharedSteps = 16;  // steps of gamma one workgroup can share (D <= 8192)
constexpr int kMaxWideRows = 4;      // rows whose scales one wide store covers

// Cache policy of the full-line output stores (residual_out, norm_out, codes):
// sc1 | nt, written through L2 as streaming data.  Scale words keep the
// default policy so that L2 merges neighbouring rows' words into whole sectors.
constexpr int kStoreAux = 18;

// Kernel arguments (element pointers; the kernels build buffer descriptors).
// Kept to 80 bytes: the host cost of a launch grows with the argument size
// (measured 2.5 us for 16 bytes, 3.7 us for 176 on this runtime), and
// decode-sized calls are bound by it.  The small mapping fields share cfg.
struct KArgs {
  const uint16_t* x;
  const uint16_t* res;
  const uint16_t* gamma;
  uint16_t* res_out;
  uint16_t* norm_out;  // nullptr: 3-output form
  uint8_t* q;
  uint8_t* scale;      // fp32 (SF_F32) or uint8 (SF_UE8M0) words
  int32_t M;           // rows (< 2^31)
  int32_t D;
  int32_t groups;      // D / G
  float eps;
  // bits 0-4 waves per row, 5-9 row groups per workgroup, 10-16 remap (see
  // tile_of_block), 17-19 log2(remap) when remap >= 2, 20 column-major scales
  // ([groups, M]), 21 wide scale stores allowed (RG_WIDE_SCALES: M % rpb == 0
  // and the scale pointer aligned to rpb words).
  uint32_t cfg;
  int32_t wpr_magic;   // ceil(2^16 / wpr): wave / wpr == (wave * wpr_magic) >> 16 for wave < 64

  __host__ __device__ int wpr() const { return (int)(cfg & 31u); }
  __host__ __device__ int rpb() const { return (int)((cfg >> 5) & 31u); }
  __host__ __device__ int remap() const { return (int)((cfg >> 10) & 127u); }
  __host__ __device__ int remap_shift() const { return (int)((cfg >> 17) & 7u); }
  __host__ __device__ int col_major() const { return (int)((cfg >> 20) & 1u); }
  __host__ __device__ int wide_ok() const { return (int)((cfg >> 21) & 1u); }
  // Each field is masked to its width, so an out-of-range value cannot reach
  // the neighbouring fields (the host passes only validated values).
  __host__ __device__ static uint32_t pack_cfg(int wpr, int rpb, int remap, int remap_shift,
                                               int col_major, int wide_ok) {
    return ((uint32_t)wpr & 31u) | (((uint32_t)rpb & 31u) << 5) |
           (((uint32_t)remap & 127u) << 10) | (((uint32_t)remap_shift & 7u) << 17) |
           (((uint32_t)col_major & 1u) << 20) | (((uint32_t)wide_ok & 1u) << 21);
  }
};
static_assert(sizeof(KArgs) == 80, "kernel argument size");

// Multi-input form (fagq_rows_parts): x = x_parts[0] + ... + x_parts[nparts - 1].
struct PArgs {
  KArgs k;
  int32_t nparts;
  const uint16_t* xparts[kMaxParts];
};

// ---------------------------------------------------------------- helpers

__device__ __forceinline__ float bf16_lo(uint32_t v) { return __uint_as_float(v << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t v) { return __uint_as_float(v & 0xffff0000u); }

// Raw buffer descriptor over [base, base + bytes): dword3 = 0x00020000 is the
// gfx9 raw-buffer word (32-bit data format, no swizzle); stride 0.
typedef __amdgpu_buffer_rsrc_t rsrc_t;
constexpr int kRsrcWord3 = 0x00020000;
constexpr int kNonTemporal = 2;     // cache-policy bit NT (gfx940 family)

__device__ __forceinline__ rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                           kRsrcWord3);
}

// Two fp32 -> packed bf16x2, round to nearest even (v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  typedef float f32x2 __attribute__((ext_vector_type(2)));
  typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
  f32x2 v = {lo, hi};
  bf16x2 b = __builtin_convertvector(v, bf16x2);
  return __builtin_bit_cast(uint32_t, b);
}

// Element types of the operator's tensors.
enum ElemType { ET_BF16 = 0, ET_F16 = 1, ET_F32 = 2 };

__device__ __forceinline__ float f16_lo(uint32_t v) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)(v & 0xffffu));
}
__device__ __forceinline__ float f16_hi(uint32_t v) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)(v >> 16));
}

// Two fp32 -> packed fp16x2, round to nearest even (v_cvt_pk_f16_f32).
__device__ __forceinline__ uint32_t pack_f16x2(float lo, float hi) {
  typedef float f32x2 __attribute__((ext_vector_type(2)));
  typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
  f32x2 v = {lo, hi};
  f16x2 h = __builtin_convertvector(v, f16x2);
  return __builtin_bit_cast(uint32_t, h);
}

// The low / high element of a word holding two 16-bit elements of type E
// (ET_BF16 or ET_F16) as fp32, and two fp32 values packed as E.
template <int E>
__device__ __forceinline__ float lo16(uint32_t v) {
  static_assert(E == ET_BF16 || E == ET_F16, "16-bit element type");
  if constexpr (E == ET_F16) return f16_lo(v);
  else return bf16_lo(v);
}
template <int E>
__device__ __forceinline__ float hi16(uint32_t v) {
  static_assert(E == ET_BF16 || E == ET_F16, "16-bit element type");
  if constexpr (E == ET_F16) return f16_hi(v);
  else return bf16_hi(v);
}
template <int E>
__device__ __forceinline__ uint32_t pack16(float lo, float hi) {
  static_assert(E == ET_BF16 || E == ET_F16, "16-bit element type");
  if constexpr (E == ET_F16) return pack_f16x2(lo, hi);
  else return pack_bf16x2(lo, hi);
}

template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xf, 0xf, false);
}

template <int CTRL>
__device__ __forceinline__ uint32_t umax_dpp(uint32_t m) {
  const uint32_t o = dpp_u32<CTRL>(m);
  return m > o ? m : o;
}

// Maximum of a non-negative fp32 (as bits) over the LPG consecutive lanes of
// one group; every lane of the group receives the result.  Non-negative fp32
// values order like their bit patterns, so the DPP steps are integer maxima
// (v_max_u32 with a DPP source, no NaN canonicalisation).
template <int LPG>
__device__ __forceinline__ uint32_t group_max_bits(uint32_t m) {
  static_assert(LPG == 8 || LPG == 16 || LPG == 32, "lanes per group");
  m = umax_dpp<0xB1>(m);    // quad_perm [1,0,3,2]
  m = umax_dpp<0x4E>(m);    // quad_perm [2,3,0,1]
  m = umax_dpp<0x141>(m);   // row_half_mirror: lanes i <-> 7-i
  if constexpr (LPG >= 16) m = umax_dpp<0x140>(m);   // row_mirror: i <-> 15-i
  if constexpr (LPG >= 32) {
    // Both lanes of a swapped pair hold the maximum of their own row after the
    // steps above; max() of the pair is the 32-lane maximum.
    const auto r = __builtin_amdgcn_permlane16_swap(m, m, false, false);
    m = r[0] > r[1] ? r[0] : r[1];
  }
  return m;
}

template <int CTRL>
__device__ __forceinline__ double dpp_f64(double v) {
  const uint64_t u = __builtin_bit_cast(uint64_t, v);
  const uint64_t o = (uint64_t)dpp_u32<CTRL>((uint32_t)u) |
                     ((uint64_t)dpp_u32<CTRL>((uint32_t)(u >> 32)) << 32);
  return __builtin_bit_cast(double, o);
}

// Sum over the 64 lanes; every lane receives the same value (each step adds
// a lane's value to its partner's, and fp addition is commutative, so both
// partners compute the identical sum).
__device__ __forceinline__ double wave_sum(double v) {
  v += dpp_f64<0xB1>(v);    // quad_perm [1,0,3,2]
  v += dpp_f64<0x4E>(v);    // quad_perm [2,3,0,1]
  v += dpp_f64<0x141>(v);   // row_half_mirror
  v += dpp_f64<0x140>(v);   // row_mirror: every lane holds its 16-lane row sum
  {
    const uint64_t u = __builtin_bit_cast(uint64_t, v);
    const auto lo = __builtin_amdgcn_permlane16_swap((uint32_t)u, (uint32_t)u, false, false);
    const auto hi = __builtin_amdgcn_permlane16_swap((uint32_t)(u >> 32), (uint32_t)(u >> 32), false, false);
    v = __builtin_bit_cast(double, (uint64_t)lo[0] | ((uint64_t)hi[0] << 32)) +
        __builtin_bit_cast(double, (uint64_t)lo[1] | ((uint64_t)hi[1] << 32));
  }
  {
    const uint64_t u = __builtin_bit_cast(uint64_t, v);
    const auto lo = __builtin_amdgcn_permlane32_swap((uint32_t)u, (uint32_t)u, false, false);
    const auto hi = __builtin_amdgcn_permlane32_swap((uint32_t)(u >> 32), (uint32_t)(u >> 32), false, false);
    v = __builtin_bit_cast(double, (uint64_t)lo[0] | ((uint64_t)hi[0] << 32)) +
        __builtin_bit_cast(double, (uint64_t)lo[1] | ((uint64_t)hi[1] << 32));
  }
  return v;
}

// Workgroup barrier whose fences cover LDS only: global stores issued before
// it need not have completed.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// inv_rms = fp32(1 / sqrt(fp32(fp32(sumsq) / D) + eps)), the square root and
// the reciprocal in IEEE double precision.
__device__ __forceinline__ float row_inv_rms(double ss, int D, float eps) {
  const float sumsq = (float)ss;
  const float mean = sumsq / (float)D;
  return (float)(1.0 / __builtin_sqrt((double)(mean + eps)));
}

// Workgroups are dispatched round-robin over the 8 XCDs (workgroup b runs on
// XCD b % 8), and each XCD has its own L2.  Row-tile order:
//   remap 0: tile = b (dispatch order);
//   remap 1: each XCD gets one contiguous range of tiles;
//   remap n >= 2: in every chunk of 8 * n consecutive workgroups, XCD x gets
//     the n consecutive tiles starting at x * n (a partial last chunk keeps
//     dispatch order).  The tiles in flight stay one contiguous window, and
//     n neighbouring rows' column-major scale words meet in one L2, so they
//     leave it as one full 32-byte write instead of n partial ones.
//   All three are computed with shifts and masks (the chunk is a power of
//   two) and one is selected, so the prologue has no branch and no integer
//   division.
__device__ __forceinline__ int tile_of_block(int b, int nb, int remap, int remap_shift) {
  const int x = b & 7, i = b >> 3, per = nb >> 3, rem = nb & 7;
  const int contiguous = x * per + (x < rem ? x : rem) + i;
  const int cs = 3 + remap_shift;                       // log2(chunk), chunk = 8 * remap
  const int c = b >> cs;
  const int w = b & ((1 << cs) - 1);
  const int chunked = ((c + 1) << cs) > nb ? b : (c << cs) + ((w & 7) << remap_shift) + (w >> 3);
  return remap == 0 ? b : remap == 1 ? contiguous : chunked;
}

// ceil(log2(s)) for a positive normal fp32 s, exactly, from its bits.
__device__ __forceinline__ int ceil_log2_bits(float s) {
  const uint32_t b = __float_as_uint(s);
  return (int)(b >> 23) - 127 + ((b & 0x7fffffu) != 0u);
}

// Eight clamped fp32 values -> eight codes (little-endian bytes).
template <int QF>
__device__ __forceinline__ u32x2 encode8(const float (&t)[8]) {
  u32x2 out;
  if constexpr (QF == QF_FP8) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      int p = __builtin_amdgcn_cvt_pk_fp8_f32(t[4 * h + 0], t[4 * h + 1], 0, false);
      p = __builtin_amdgcn_cvt_pk_fp8_f32(t[4 * h + 2], t[4 * h + 3], p, true);
      out[h] = (uint32_t)p;
    }
  } else {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      int iv[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float v = (QF == QF_I8_RNE) ? __builtin_rintf(t[4 * h + j]) : t[4 * h + j];
        iv[j] = (int)v;   // v_cvt_i32_f32: truncation toward zero
      }
      const uint32_t lo = __builtin_amdgcn_perm((uint32_t)iv[1], (uint32_t)iv[0], 0x0c0c0400u);
      const uint32_t hi = __builtin_amdgcn_perm((uint32_t)iv[3], (uint32_t)iv[2], 0x0c0c0400u);
      out[h] = __builtin_amdgcn_perm(hi, lo, 0x05040100u);
    }
  }
  return out;
}

// Scale addressing of one wave, shared by the kernels and the host-side
// diagnostic that checks it.  The wave's scale descriptor starts at the
// scale of its first group g0 = c0 / G and ends just after the row's last
// group: column-major scale[g * M + row] -> span (ng - 1) * M + 1 words,
// row-major scale[row * groups + g] -> span ng words, ng = groups - g0.
struct ScaleSpan {
  int64_t base;          // element index of the descriptor's first word
  uint32_t bytes;        // descriptor size in bytes
  uint32_t ngroups;      // groups of the row at or after g0 (0: none)
  uint32_t gstride;      // byte distance between consecutive groups of the row
};

__host__ __device__ inline ScaleSpan scale_span(int64_t M, int32_t groups, int col_major,
                                                uint32_t sb, int64_t row, bool row_ok,
                                                int g0, bool cols_ok) {
  ScaleSpan r;
  const int64_t rr = row_ok ? row : 0;
  const uint32_t ng = row_ok && cols_ok ? (uint32_t)(groups - g0) : 0u;
  r.base = col_major ? (int64_t)g0 * M + rr : rr * (int64_t)groups + g0;
  const uint32_t span = col_major ? (ng ? (uint32_t)((int64_t)(ng - 1) * M + 1) : 0u) : ng;
  r.bytes = span * sb;
  r.ngroups = ng;
  r.gstride = col_major ? (uint32_t)(M * (int64_t)sb) : sb;
  return r;
}

// Byte offset (within the wave's scale descriptor) of the scale word that
// lane group gl stores at step k.  Groups past the row's end get 0xffffffff,
// which no descriptor reaches (scale spans are validated below 2^32 - 16), so
// their stores are dropped; their in-range product g * gstride could wrap
// past 2^32 into the descriptor.
__host__ __device__ inline uint32_t scale_lane_offset(uint32_t gl, uint32_t k,
                                                      uint32_t groups_per_step,
                                                      uint32_t ngroups, uint32_t gstride) {
  const uint32_t g = gl + k * groups_per_step;
  return g < ngroups ? g * gstride : 0xffffffffu;
}

// ---------------------------------------------------------------- kernel

// Row-invariant per-wave geometry.
struct WaveCtx {
  int lane;
  int c0;          // first column of this wave
  uint32_t cols;   // columns of the row at or after c0 (0 if none)
  int gl;          // group index of this lane within a step
};

// Descriptors of one row for one wave.
struct RowRsrc {
  rsrc_t x, res, res_out, norm, q, scale;
  uint32_t ngroups;      // groups of the row this wave's scale descriptor covers
  uint32_t gstride;      // byte distance between consecutive groups' scales
};

// The input descriptors (x, residual) are built first and their loads
// issued before the output descriptors are computed.
__device__ __forceinline__ void row_rsrc_in(const KArgs& a, const WaveCtx& w, int64_t row,
                                            RowRsrc& r) {
  const bool ok = row < a.M;
  const int64_t e = (ok ? row : 0) * (int64_t)a.D + w.c0;
  const uint32_t cols = ok ? w.cols : 0u;
  r.x = make_rsrc(a.x + e, cols * 2u);
  r.res = make_rsrc(a.res + e, cols * 2u);
}

template <int SF, bool NORM>
__device__ __forceinline__ void row_rsrc_out(const KArgs& a, const WaveCtx& w, int64_t row, int G,
                                             RowRsrc& r) {
  constexpr uint32_t sb = SF == SF_F32 ? 4u : 1u;
  const bool ok = row < a.M;
  const int64_t rr = ok ? row : 0;
  const int64_t e = rr * (int64_t)a.D + w.c0;
  const uint32_t cols = ok ? w.cols : 0u;
  r.res_out = make_rsrc(a.res_out + e, cols * 2u);
  if constexpr (NORM) r.norm = make_rsrc(a.norm_out + e, cols * 2u);
  r.q = make_rsrc(a.q + e, cols);
  const ScaleSpan sp = scale_span(a.M, a.groups, a.col_major(), sb, row, ok, w.c0 / G, w.cols != 0);
  r.scale = make_rsrc(a.scale + sp.base * sb, sp.bytes);
  r.ngroups = sp.ngroups;
  r.gstride = sp.gstride;
}

// Phase 1 for one row: issue the loads of x and residual for NS steps.
template <int NS>
__device__ __forceinline__ void load_row(const RowRsrc& r, int lane, u32x4 (&xv)[NS],
                                         u32x4 (&rv)[NS]) {
#pragma unroll
  for (int k = 0; k < NS; ++k) {
    xv[k] = __builtin_amdgcn_raw_buffer_load_b128(r.x, lane * 16 + k * 1024, 0, kNonTemporal);
    rv[k] = __builtin_amdgcn_raw_buffer_load_b128(r.res, lane * 16 + k * 1024, 0, kNonTemporal);
  }
}

// Gamma for this wave's columns (an L2 hit), NS steps.
template <int NS>
__device__ __forceinline__ void load_gamma(const KArgs& a, const WaveCtx& w, int lane,
                                           u32x4 (&gv)[NS]) {
  const rsrc_t rg = make_rsrc(a.gamma + w.c0, w.cols * 2u);
#pragma unroll
  for (int k = 0; k < NS; ++k)
    gv[k] = __builtin_amdgcn_raw_buffer_load_b128(rg, lane * 16 + k * 1024, 0, 0);
}

// Phase 2a for one row: r = x + residual into rw, the fp64 sum of squares, and
// the residual_out stores (after every use of the loaded data).  xs holds x in
// fp32 (one 16-bit tensor, or the fp32 sum of the partial tensors in the
// multi-input form); residual and residual_out have element type E16.
template <int NS, int E16 = ET_BF16>
__device__ __forceinline__ double row_sum(const RowRsrc& rr, int lane, const float (&xs)[NS][8],
                                          const u32x4 (&rv)[NS], float (&rw)[NS][8]) {
  double ss = 0.0;
  u32x4 ro[NS];
#pragma unroll
  for (int k = 0; k < NS; ++k) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      rw[k][2 * j] = xs[k][2 * j] + lo16<E16>(rv[k][j]);
      rw[k][2 * j + 1] = xs[k][2 * j + 1] + hi16<E16>(rv[k][j]);
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const double rd = (double)rw[k][j];
      ss = __builtin_fma(rd, rd, ss);   // r^2 is exact in fp64
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) ro[k][j] = pack16<E16>(rw[k][2 * j], rw[k][2 * j + 1]);
  }
#pragma unroll
  for (int k = 0; k < NS; ++k)
    __builtin_amdgcn_raw_buffer_store_b128(ro[k], rr.res_out, lane * 16 + k * 1024, 0, kStoreAux);
  return ss;
}

// Phase 2b: w = r * gamma in place (rw holds r on entry, w on exit) and the
// group maxima of |w|.
template <int NS, int LPG, int E16 = ET_BF16>
__device__ __forceinline__ void row_weight(float (&rw)[NS][8], const u32x4 (&gv)[NS],
                                           uint32_t (&gmax)[NS]) {
#pragma unroll
  for (int k = 0; k < NS; ++k) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      rw[k][2 * j] = rw[k][2 * j] * lo16<E16>(gv[k][j]);
      rw[k][2 * j + 1] = rw[k][2 * j + 1] * hi16<E16>(gv[k][j]);
    }
    float m = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; ++j) m = __builtin_fmaxf(m, __builtin_fabsf(rw[k][j]));
    gmax[k] = group_max_bits<LPG>(__float_as_uint(m));
  }
}

template <int NS, int E16 = ET_BF16>
__device__ __forceinline__ void unpack_x(const u32x4 (&xv)[NS], float (&xs)[NS][8]) {
#pragma unroll
  for (int k = 0; k < NS; ++k)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      xs[k][2 * j] = lo16<E16>(xv[k][j]);
      xs[k][2 * j + 1] = hi16<E16>(xv[k][j]);
    }
}

// Multi-input form, phase 1: the row's partial tensors of x (the same row
// and columns of each) and residual.  Parts past nparts are not loaded.
template <int NS>
__device__ __forceinline__ void load_row_parts(const PArgs& pa, const WaveCtx& w, int64_t row,
                                               const RowRsrc& rr, int lane,
                                               u32x4 (&xv)[kMaxParts][NS], u32x4 (&rv)[NS]) {
  const KArgs& a = pa.k;
  const bool ok = row < a.M;
  const int64_t e = (ok ? row : 0) * (int64_t)a.D + w.c0;
  const uint32_t cols = ok ? w.cols : 0u;
#pragma unroll
  for (int p = 0; p < kMaxParts; ++p) {
    if (p < pa.nparts) {
      const rsrc_t rp = make_rsrc(pa.xparts[p] + e, cols * 2u);
#pragma unroll
      for (int k = 0; k < NS; ++k)
        xv[p][k] = __builtin_amdgcn_raw_buffer_load_b128(rp, lane * 16 + k * 1024, 0, kNonTemporal);
    } else {
#pragma unroll
      for (int k = 0; k < NS; ++k) xv[p][k] = u32x4{0u, 0u, 0u, 0u};
    }
  }
#pragma unroll
  for (int k = 0; k < NS; ++k)
    rv[k] = __builtin_amdgcn_raw_buffer_load_b128(rr.res, lane * 16 + k * 1024, 0, kNonTemporal);
}

// x = ((x_0 + x_1) + ... + x_{nparts-1}) in fp32, in part order.
template <int NS>
__device__ __forceinline__ void sum_parts(int nparts, const u32x4 (&xv)[kMaxParts][NS],
                                          float (&xs)[NS][8]) {
#pragma unroll
  for (int k = 0; k < NS; ++k)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      xs[k][2 * j] = bf16_lo(xv[0][k][j]);
      xs[k][2 * j + 1] = bf16_hi(xv[0][k][j]);
    }
#pragma unroll
  for (int p = 1; p < kMaxParts; ++p) {
    if (p < nparts) {
#pragma unroll
      for (int k = 0; k < NS; ++k)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          xs[k][2 * j] = xs[k][2 * j] + bf16_lo(xv[p][k][j]);
          xs[k][2 * j + 1] = xs[k][2 * j + 1] + bf16_hi(xv[p][k][j]);
        }
    }
  }
}

// The scale of one group from its |w| maximum: fp32 s, or for UE8M0 the
// exponent e = ceil(log2(s)) (at most 127).
template <int SF>
__device__ __forceinline__ float group_scale(uint32_t gmax_bits, float inv_q, int& e) {
  const float s = __builtin_fmaxf(__uint_as_float(gmax_bits) * inv_q, 1.0e-12f);
  if constexpr (SF == SF_UE8M0) {
    e = ceil_log2_bits(s);
    e = e > 127 ? 127 : e;
  }
  return s;
}

// ---------------------------------------------------------------- element types

// Element types of the tensors around the operator.  fagq_rows reads and
// writes one 16-bit type (bf16, or fp16 for the typed form's fp16 family);
// the typed kernel (fagq_rows_typed) serves the families with an fp32 tensor:
// one element type for the activation tensors (x, gamma, norm_out) and one for
// the residual stream (residual, residual_out).  Both convert every load to
// fp32 and every store from fp32 (round to nearest even), as the reference's
// kernels do (task01.py:88-89, :93-94 loads; :91, :118 stores).

// Type families of the typed form: (activation type, residual-stream type).
// TF_F16 runs fagq_rows<..., ET_F16>, the others fagq_rows_typed.
enum TypeFamily { TF_F16 = 0, TF_BF16_R32 = 1, TF_F16_R32 = 2, TF_F32 = 3 };
constexpr int kNumTypeFamilies = 4;

template <int TF>
struct Family {
  static constexpr int A = TF == TF_F16 || TF == TF_F16_R32 ? ET_F16
                           : TF == TF_BF16_R32            ? ET_BF16
                                                          : ET_F32;
  static constexpr int R = TF == TF_F16 ? ET_F16 : ET_F32;
};

template <int ET>
constexpr uint32_t elem_bytes() {
  return ET == ET_F32 ? 4u : 2u;
}

// A lane's 8 elements of one step: one 16-byte word for 2-byte types, two for
// fp32.  2-byte types: lane l loads elements 8l..8l+7 of the step (bytes 16l..,
// the wave's 64 loads one contiguous 1 KB).  fp32: the wave reads the step's
// 2 KB as two contiguous 1 KB loads (lane l: 16-byte chunks l and 64 + l), and
// lane_order() hands each lane its own chunks 2l and 2l + 1 through the wave's
// LDS stage.  A lane-ordered fp32 load would stride 32 bytes per lane and
// touch every 32-byte sector in two halves; on stores that means partial-sector
// writes to HBM.
template <int ET>
struct Vec8 {
  u32x4 v[ET == ET_F32 ? 2 : 1];
};

// 2 KB of LDS per wave: fp32 chunks on their way between wave order and lane
// order.  A wave's LDS accesses execute in program order, so the hardware
// needs no barrier between its transposes; the compiler, which reasons about
// one lane, must not move a lane's read of another lane's slot across the
// write of that slot (stage_sync between the two halves of each exchange).
typedef u32x4 Stage[128];

__device__ __forceinline__ void stage_sync() {
  __builtin_amdgcn_wave_barrier();
  asm volatile("" ::: "memory");
}

template <int ET, int AUX>
__device__ __forceinline__ Vec8<ET> load_elems8(const rsrc_t& rs, int lane, int k) {
  Vec8<ET> r;
  if constexpr (ET == ET_F32) {
#pragma unroll
    for (int h = 0; h < 2; ++h)
      r.v[h] = __builtin_amdgcn_raw_buffer_load_b128(rs, lane * 16 + h * 1024 + k * kStepCols * 4,
                                                     0, AUX);
  } else {
    r.v[0] = __builtin_amdgcn_raw_buffer_load_b128(rs, lane * 16 + k * kStepCols * 2, 0, AUX);
  }
  return r;
}

// fp32 step as loaded (chunks l, 64 + l) -> lane order (chunks 2l, 2l + 1).
template <int ET>
__device__ __forceinline__ void lane_order(Vec8<ET>& p, int lane, Stage& st) {
  if constexpr (ET == ET_F32) {
    st[lane] = p.v[0];
    st[64 + lane] = p.v[1];
    stage_sync();
    p.v[0] = st[2 * lane];
    p.v[1] = st[2 * lane + 1];
    stage_sync();
  }
}

template <int ET>
__device__ __forceinline__ void unpack_elems8(const Vec8<ET>& p, float (&f)[8]) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    if constexpr (ET == ET_BF16) {
      f[2 * j] = bf16_lo(p.v[0][j]);
      f[2 * j + 1] = bf16_hi(p.v[0][j]);
    } else if constexpr (ET == ET_F16) {
      f[2 * j] = f16_lo(p.v[0][j]);
      f[2 * j + 1] = f16_hi(p.v[0][j]);
    } else {
      f[j] = __uint_as_float(p.v[0][j]);
      f[4 + j] = __uint_as_float(p.v[1][j]);
    }
  }
}

// Stores a lane's 8 fp32 values of step k as ET (streaming stores); fp32
// passes through the wave's LDS stage to leave as two contiguous 1 KB stores
// (st is used for fp32 only).
template <int ET>
__device__ __forceinline__ void store_elems8(const rsrc_t& rs, int lane, int k,
                                             const float (&f)[8], Stage* st = nullptr) {
  if constexpr (ET == ET_F32) {
    (*st)[2 * lane] = u32x4{__float_as_uint(f[0]), __float_as_uint(f[1]), __float_as_uint(f[2]),
                            __float_as_uint(f[3])};
    (*st)[2 * lane + 1] = u32x4{__float_as_uint(f[4]), __float_as_uint(f[5]),
                                __float_as_uint(f[6]), __float_as_uint(f[7])};
    stage_sync();
    const u32x4 c0 = (*st)[lane], c1 = (*st)[64 + lane];
    stage_sync();
    __builtin_amdgcn_raw_buffer_store_b128(c0, rs, lane * 16 + k * kStepCols * 4, 0, kStoreAux);
    __builtin_amdgcn_raw_buffer_store_b128(c1, rs, lane * 16 + 1024 + k * kStepCols * 4, 0,
                                           kStoreAux);
  } else {
    u32x4 o;
#pragma unroll
    for (int j = 0; j < 4; ++j)
      o[j] = ET == ET_BF16 ? pack_bf16x2(f[2 * j], f[2 * j + 1]) : pack_f16x2(f[2 * j], f[2 * j + 1]);
    __builtin_amdgcn_raw_buffer_store_b128(o, rs, lane * 16 + k * kStepCols * 2, 0, kStoreAux);
  }
}

// Phase 4 for one row: codes, optional norm_out and, with STORE_SCALES, the
// scales (every lane of a group stores the group's scale to the same
// address, one write after coalescing; groups past the row end get an
// offset outside the descriptor and are dropped).
template <int NS, int LPG, int QF, int SF, bool NORM, bool STORE_SCALES = true,
          int NET = ET_BF16>
__device__ __forceinline__ void row_out(const RowRsrc& rr, int lane, uint32_t gl,
                                        const float (&w)[NS][8], const uint32_t (&gmax)[NS],
                                        float inv, float inv_q, Stage* st = nullptr) {
  constexpr uint32_t GPS = kStepCols / (LPG * 8);
#pragma unroll
  for (int k = 0; k < NS; ++k) {
    int e = 0;
    const float s = group_scale<SF>(gmax[k], inv_q, e);
    float mul = 0.0f;
    if constexpr (SF == SF_F32) mul = 1.0f / s;
    // No clamp to [-QMAX, QMAX]: for finite inputs |t| <= QMAX * (1 + 5 * 2^-24)
    // (|n| <= gmax * inv and s >= gmax * inv / QMAX, each up to a few
    // roundings), and fp8 rounds everything below 464 to at most 448, int8
    // rounding and truncation give at most 127, so the reference's clamp never
    // changes a code.
    float n[8], t[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      n[j] = w[k][j] * inv;
      t[j] = (SF == SF_F32) ? n[j] * mul : __builtin_ldexpf(n[j], -e);
    }
    if constexpr (NORM) store_elems8<NET>(rr.norm, lane, k, n, st);   // norm_out's element type
    const u32x2 codes = encode8<QF>(t);
    __builtin_amdgcn_raw_buffer_store_b64(codes, rr.q, lane * 8 + k * 512, 0, kStoreAux);
    if constexpr (STORE_SCALES) {
      const uint32_t off = scale_lane_offset(gl, (uint32_t)k, GPS, rr.ngroups, rr.gstride);
      if constexpr (SF == SF_F32)
        __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(s), rr.scale, off, 0, 0);
      else
        __builtin_amdgcn_raw_buffer_store_b8((uint8_t)(e + 127), rr.scale, off, 0, 0);
    }
  }
}

// Phase 3: a wave's partial sum of squares -> the row's inv_rms and
// inv_rms / QMAX.  With several waves per row, the row's first wave adds the
// partial sums (in wave order) and evaluates inv_rms once; a second barrier
// hands it to the others.  Both barriers are fenced for LDS only, so no
// global store has to complete before them.  Every wave of the workgroup
// calls this (the barriers are workgroup-wide).
template <int QF>
__device__ __forceinline__ void row_scale(double ss, const KArgs& a, int wave, int rib, int part,
                                          int wpr, int lane, double* s_part, float (*s_inv)[2],
                                          float& inv, float& inv_q) {
  constexpr float QMAX = (QF == QF_FP8) ? 448.0f : 127.0f;
  ss = wave_sum(ss);
  if (wpr > 1) {
    if (lane == 0) s_part[wave] = ss;
    lds_barrier();
    if (part == 0) {
      double t = 0.0;
      for (int p = 0; p < wpr; ++p) t += s_part[rib * wpr + p];
      const float v = row_inv_rms(t, a.D, a.eps);
      if (lane == 0) {
        s_inv[rib][0] = v;
        s_inv[rib][1] = v / QMAX;
      }
    }
    lds_barrier();
    inv = s_inv[rib][0];
    inv_q = s_inv[rib][1];
  } else {
    inv = row_inv_rms(ss, a.D, a.eps);
    inv_q = inv / QMAX;
  }
}

// Workgroup = rpb row groups of wpr waves; row group j of workgroup b owns
// row b * rpb + j.  MODE (RowGroupMode) selects how the row groups share
// gamma and store the scales:
//   RG_INDEPENDENT: each wave loads its gamma slice and computes w = r * gamma
//     before the row's reduction; each row group stores its own scales.
//   RG_SHARED_GAMMA: only row group 0 loads gamma; it leaves its slices in
//     LDS, and the other row groups compute w after the first barrier (the
//     values and the operation order are the same, only the time differs).
//   RG_WIDE_SCALES: as RG_SHARED_GAMMA, and the group maxima of every row go
//     to LDS, so that after the second barrier row group 0 evaluates the
//     scales of all rpb rows (the same expression each row would evaluate) and
//     stores each group's rpb consecutive column-major words with one store.
//     A workgroup whose rows would pass M, or a call whose scale pointer or M
//     does not allow the wide alignment (wide_ok == 0), stores row by row.
// E16: element type of x, residual, gamma, residual_out and norm_out
// (ET_BF16, or ET_F16 for the typed form's fp16 tensors).
template <int NS, int LPG, int QF, int SF, bool NORM, int MODE, int E16 = ET_BF16>
__global__ void __launch_bounds__(1024)
fagq_rows(const KArgs a) {
  static_assert(NS >= 1 && NS <= kMaxStepsPerWave, "steps per wave");
  static_assert(MODE >= 0 && MODE < kNumModes, "row-group mode");
  constexpr int G = LPG * 8;
  constexpr int GPS = kStepCols / G;    // groups per step
  constexpr uint32_t sb = SF == SF_F32 ? 4u : 1u;
  constexpr bool SHARED = MODE != RG_INDEPENDENT;
  constexpr bool WIDE = MODE == RG_WIDE_SCALES;
  constexpr float QMAX = (QF == QF_FP8) ? 448.0f : 127.0f;
  __shared__ double s_part[kMaxWavesPerBlock];
  __shared__ float s_inv[kMaxWavesPerBlock][2];
  // Shared modes only (the arrays are not allocated otherwise): gamma slices
  // [step of the row][lane], and the group maxima [row group][group].
  __shared__ u32x4 s_gamma[SHARED ? kMaxSharedSteps * 64 : 1];
  __shared__ uint32_t s_gmax[WIDE ? kMaxWideRows : 1][WIDE ? kMaxSharedSteps * GPS : 1];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wpr = a.wpr();
  const int blk = tile_of_block((int)blockIdx.x, (int)gridDim.x, a.remap(), a.remap_shift());
  // Row group within the workgroup and wave within the row (wpr * rpb waves).
  const int rib = (wave * a.wpr_magic) >> 16;
  const int part = wave - rib * wpr;
  const int64_t row0 = (int64_t)blk * a.rpb();
  const int64_t row = row0 + rib;
  WaveCtx wc;
  wc.lane = lane;
  wc.c0 = part * (NS * kStepCols);
  wc.cols = a.D > wc.c0 ? (uint32_t)(a.D - wc.c0) : 0u;
  wc.gl = lane / LPG;
  const int g0 = wc.c0 / G;

  // The row's inputs go out first, then gamma for this wave's columns (an L2
  // hit, needed at the same time), then the output descriptors are computed.
  u32x4 xv[NS], rv[NS];
  RowRsrc rr;
  row_rsrc_in(a, wc, row, rr);
  load_row<NS>(rr, lane, xv, rv);
  const bool gamma_loader = !SHARED || rib == 0;
  u32x4 gv[NS];
  if (gamma_loader) load_gamma<NS>(a, wc, lane, gv);
  row_rsrc_out<SF, NORM>(a, wc, row, G, rr);

  float w[NS][8];
  uint32_t gmax[NS];
  double ss;
  {
    float xs[NS][8];
    unpack_x<NS, E16>(xv, xs);
    ss = row_sum<NS, E16>(rr, lane, xs, rv, w);
  }
  auto publish_gmax = [&](int rg) {
    if ((lane & (LPG - 1)) == 0) {
#pragma unroll
      for (int k = 0; k < NS; ++k) {
        const int g = g0 + k * GPS + wc.gl;
        if (g < a.groups) s_gmax[rg][g] = gmax[k];
      }
    }
  };
  if (gamma_loader) {
    row_weight<NS, LPG, E16>(w, gv, gmax);
    if constexpr (SHARED) {
#pragma unroll
      for (int k = 0; k < NS; ++k) s_gamma[(part * NS + k) * 64 + lane] = gv[k];
      if constexpr (WIDE) publish_gmax(0);
    }
  }

  // The row's sum of squares: with several waves per row (or shared gamma),
  // the row's first wave adds the partial sums in wave order and evaluates
  // inv_rms once; a second barrier hands it to the others.  Both barriers
  // are fenced for LDS only, so no global store has to complete before them.
  float inv, inv_q;
  ss = wave_sum(ss);
  if (wpr > 1 || SHARED) {
    if (lane == 0) s_part[wave] = ss;
    lds_barrier();
    if (SHARED && !gamma_loader) {
#pragma unroll
      for (int k = 0; k < NS; ++k) gv[k] = s_gamma[(part * NS + k) * 64 + lane];
      row_weight<NS, LPG, E16>(w, gv, gmax);
      if constexpr (WIDE) publish_gmax(rib);
    }
    if (part == 0) {
      double t = 0.0;
      for (int p = 0; p < wpr; ++p) t += s_part[rib * wpr + p];
      const float v = row_inv_rms(t, a.D, a.eps);
      if (lane == 0) {
        s_inv[rib][0] = v;
        s_inv[rib][1] = v / QMAX;
      }
    }
    lds_barrier();
    inv = s_inv[rib][0];
    inv_q = s_inv[rib][1];
  } else {
    inv = row_inv_rms(ss, a.D, a.eps);
    inv_q = inv / QMAX;
  }

  if constexpr (WIDE) {
    const int R = a.rpb();
    const bool wide = a.wide_ok() && row0 + R <= a.M;
    if (wide) {
      row_out<NS, LPG, QF, SF, NORM, false, E16>(rr, lane, (uint32_t)wc.gl, w, gmax, inv, inv_q);
      if (rib == 0 && (lane & (LPG - 1)) == 0) {
        // Scale words g * M + row0 .. + R - 1, offsets below M * groups * sb.
        const rsrc_t rs = make_rsrc(a.scale, (uint32_t)((int64_t)a.M * a.groups * sb));
#pragma unroll
        for (int k = 0; k < NS; ++k) {
          const int g = g0 + k * GPS + wc.gl;
          if (g < a.groups) {
            uint32_t v[kMaxWideRows];
#pragma unroll
            for (int j = 0; j < kMaxWideRows; ++j) {
              v[j] = 0u;
              if (j < R) {
                int e = 0;
                const float sj = group_scale<SF>(s_gmax[j][g], s_inv[j][1], e);
                v[j] = SF == SF_F32 ? __float_as_uint(sj) : (uint32_t)(e + 127);
              }
            }
            const uint32_t off = (uint32_t)(((int64_t)g * a.M + row0) * sb);
            if constexpr (SF == SF_F32) {
              if (R == 2)
                __builtin_amdgcn_raw_buffer_store_b64(u32x2{v[0], v[1]}, rs, off, 0, 0);
              else
                __builtin_amdgcn_raw_buffer_store_b128(u32x4{v[0], v[1], v[2], v[3]}, rs, off, 0, 0);
            } else {
              if (R == 2)
                __builtin_amdgcn_raw_buffer_store_b16((uint16_t)(v[0] | (v[1] << 8)), rs, off, 0, 0);
              else
                __builtin_amdgcn_raw_buffer_store_b32(v[0] | (v[1] << 8) | (v[2] << 16) | (v[3] << 24),
                                                      rs, off, 0, 0);
            }
          }
        }
      }
    } else {
      row_out<NS, LPG, QF, SF, NORM, true, E16>(rr, lane, (uint32_t)wc.gl, w, gmax, inv, inv_q);
    }
  } else {
    row_out<NS, LPG, QF, SF, NORM, true, E16>(rr, lane, (uint32_t)wc.gl, w, gmax, inv, inv_q);
  }
}

// Multi-input form (the epilogue of a tensor-parallel reduction): x is the
// sum of nparts partial tensors, one per rank, added in fp32 in rank order
// before the residual; everything after is the operator above.  One row per
// row group, no norm_out, at most kMaxStepsParts steps per wave (the partial
// loads of a wave's steps are all in flight at once).  4-step waves hold up to
// 8 x 4 partial loads (about 200 VGPRs), so their workgroups are bounded to 8
// waves (256 VGPRs per lane).
template <int NS, int LPG, int QF, int SF>
__global__ void __launch_bounds__(NS > 2 ? 512 : 1024)
fagq_rows_parts(const PArgs pa) {
  const KArgs& a = pa.k;
  static_assert(NS >= 1 && NS <= kMaxStepsParts, "steps per wave");
  constexpr int G = LPG * 8;
  __shared__ double s_part[kMaxWavesPerBlock];
  __shared__ float s_inv[kMaxWavesPerBlock][2];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wpr = a.wpr();
  const int blk = tile_of_block((int)blockIdx.x, (int)gridDim.x, a.remap(), a.remap_shift());
  const int rib = (wave * a.wpr_magic) >> 16;
  const int part = wave - rib * wpr;
  const int64_t row = (int64_t)blk * a.rpb() + rib;
  WaveCtx wc;
  wc.lane = lane;
  wc.c0 = part * (NS * kStepCols);
  wc.cols = a.D > wc.c0 ? (uint32_t)(a.D - wc.c0) : 0u;
  wc.gl = lane / LPG;

  u32x4 xv[kMaxParts][NS], rv[NS];
  RowRsrc rr;
  row_rsrc_in(a, wc, row, rr);
  load_row_parts<NS>(pa, wc, row, rr, lane, xv, rv);
  u32x4 gv[NS];
  load_gamma<NS>(a, wc, lane, gv);
  row_rsrc_out<SF, false>(a, wc, row, G, rr);

  float w[NS][8];
  uint32_t gmax[NS];
  double ss;
  {
    float xs[NS][8];
    sum_parts<NS>(pa.nparts, xv, xs);
    ss = row_sum<NS>(rr, lane, xs, rv, w);
  }
  row_weight<NS, LPG>(w, gv, gmax);
  float inv, inv_q;
  row_scale<QF>(ss, a, wave, rib, part, wpr, lane, s_part, s_inv, inv, inv_q);
  row_out<NS, LPG, QF, SF, false>(rr, lane, (uint32_t)wc.gl, w, gmax, inv, inv_q);
}

// Typed form (fagq_launch_typed) for the families with an fp32 tensor: the
// operator with activation tensors (x, gamma, norm_out) of element type
// Family<TF>::A and a residual stream (residual, residual_out) of type
// Family<TF>::R, each converted to fp32 on load and rounded to nearest even on
// store; the arithmetic from r = x + residual on is the bf16 kernel's,
// operation for operation.  Row groups are independent (each wave loads its
// own gamma slice, each row stores its own scales); the element sizes set the
// descriptors and offsets.  (TF_F16 would also compile here; it runs
// fagq_rows with fp16 elements instead, with the bf16 operator's route.)
template <int NS, int LPG, int QF, int SF, bool NORM, int TF>
__global__ void __launch_bounds__(1024)
fagq_rows_typed(const KArgs a) {
  static_assert(NS >= 1 && NS <= kMaxStepsPerWave, "steps per wave");
  static_assert(TF >= 0 && TF < kNumTypeFamilies, "type family");
  constexpr int EA = Family<TF>::A, ER = Family<TF>::R;
  constexpr uint32_t ba = elem_bytes<EA>(), br = elem_bytes<ER>();
  constexpr int G = LPG * 8;
  constexpr uint32_t sb = SF == SF_F32 ? 4u : 1u;
  constexpr bool F32IO = EA == ET_F32 || ER == ET_F32;
  __shared__ double s_part[kMaxWavesPerBlock];
  __shared__ float s_inv[kMaxWavesPerBlock][2];
  __shared__ Stage s_stage[F32IO ? kMaxWavesPerBlock : 1];   // fp32 transposes, per wave

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  Stage& st = s_stage[F32IO ? wave : 0];
  const int wpr = a.wpr();
  const int blk = tile_of_block((int)blockIdx.x, (int)gridDim.x, a.remap(), a.remap_shift());
  const int rib = (wave * a.wpr_magic) >> 16;
  const int part = wave - rib * wpr;
  const int64_t row = (int64_t)blk * a.rpb() + rib;
  const int c0 = part * (NS * kStepCols);
  const uint32_t wcols = a.D > c0 ? (uint32_t)(a.D - c0) : 0u;
  const bool ok = row < a.M;
  const int64_t e = (ok ? row : 0) * (int64_t)a.D + c0;
  const uint32_t cols = ok ? wcols : 0u;

  RowRsrc rr;
  const uint8_t* xb = reinterpret_cast<const uint8_t*>(a.x);
  const uint8_t* rb = reinterpret_cast<const uint8_t*>(a.res);
  rr.x = make_rsrc(xb + e * ba, cols * ba);
  rr.res = make_rsrc(rb + e * br, cols * br);
  Vec8<EA> xv[NS];
  Vec8<ER> rv[NS];
#pragma unroll
  for (int k = 0; k < NS; ++k) {
    xv[k] = load_elems8<EA, kNonTemporal>(rr.x, lane, k);
    rv[k] = load_elems8<ER, kNonTemporal>(rr.res, lane, k);
  }
  const rsrc_t rg = make_rsrc(reinterpret_cast<const uint8_t*>(a.gamma) + c0 * ba, wcols * ba);
  Vec8<EA> gv[NS];
#pragma unroll
  for (int k = 0; k < NS; ++k) gv[k] = load_elems8<EA, 0>(rg, lane, k);
  rr.res_out = make_rsrc(reinterpret_cast<uint8_t*>(a.res_out) + e * br, cols * br);
  if constexpr (NORM) rr.norm = make_rsrc(reinterpret_cast<uint8_t*>(a.norm_out) + e * ba, cols * ba);
  rr.q = make_rsrc(a.q + e, cols);
  const ScaleSpan sp = scale_span(a.M, a.groups, a.col_major(), sb, row, ok, c0 / G, wcols != 0);
  rr.scale = make_rsrc(a.scale + sp.base * sb, sp.bytes);
  rr.ngroups = sp.ngroups;
  rr.gstride = sp.gstride;

  // r = x + residual, residual_out, the fp64 sum of squares, w = r * gamma and
  // the group maxima, in the bf16 kernel's order.
  float w[NS][8];
  uint32_t gmax[NS];
  double ss = 0.0;
#pragma unroll
  for (int k = 0; k < NS; ++k) {
    float xs[8], rs[8];
    lane_order<EA>(xv[k], lane, st);
    lane_order<ER>(rv[k], lane, st);
    unpack_elems8<EA>(xv[k], xs);
    unpack_elems8<ER>(rv[k], rs);
#pragma unroll
    for (int j = 0; j < 8; ++j) w[k][j] = xs[j] + rs[j];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const double rd = (double)w[k][j];
      ss = __builtin_fma(rd, rd, ss);
    }
  }
#pragma unroll
  for (int k = 0; k < NS; ++k) store_elems8<ER>(rr.res_out, lane, k, w[k], &st);
#pragma unroll
  for (int k = 0; k < NS; ++k) {
    float gs[8];
    lane_order<EA>(gv[k], lane, st);
    unpack_elems8<EA>(gv[k], gs);
#pragma unroll
    for (int j = 0; j < 8; ++j) w[k][j] = w[k][j] * gs[j];
    float m = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; ++j) m = __builtin_fmaxf(m, __builtin_fabsf(w[k][j]));
    gmax[k] = group_max_bits<LPG>(__float_as_uint(m));
  }
  float inv, inv_q;
  row_scale<QF>(ss, a, wave, rib, part, wpr, lane, s_part, s_inv, inv, inv_q);
  row_out<NS, LPG, QF, SF, NORM, true, EA>(rr, lane, (uint32_t)(lane / LPG), w, gmax, inv, inv_q,
                                           &st);
}

// ---------------------------------------------------------------- diagnostics

// Encodes already-scaled fp32 values with the same device encoder as the
// operator, 8 per thread, n % 8 == 0.  CLAMP applies the reference's clamp to
// [-QMAX, QMAX] first; without it the values reach the encoder as the
// operator's kernels pass them (they skip the clamp, see row_out).
template <int QF, bool CLAMP>
__global__ void __launch_bounds__(256) fagq_encode(const float* __restrict__ in,
                                                   u32x2* __restrict__ out, int64_t n8) {
  constexpr float QMAX = (QF == QF_FP8) ? 448.0f : 127.0f;
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n8) return;
  float t[8];
#pragma unroll
  for (int j = 0; j < 8; ++j)
    t[j] = CLAMP ? __builtin_fminf(__builtin_fmaxf(in[i * 8 + j], -QMAX), QMAX) : in[i * 8 + j];
  out[i] = encode8<QF>(t);
}

}  // namespace fagq
