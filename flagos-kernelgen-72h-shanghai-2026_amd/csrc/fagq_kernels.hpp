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
// lanes = one DPP row for G = 128), so a group maximum is a 2..5-step DPP
// reduction that never leaves the wave.
//
// A wave owns NS consecutive steps of one row and keeps r*gamma for all of
// them in VGPRs (8*NS floats per lane), so every input byte is read from HBM
// once and no intermediate is written.  waves_per_row > 1 splits a row over
// several waves of one workgroup; only the fp64 partial sum of squares then
// crosses waves, through LDS, with one barrier.
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

// Kernel arguments.  Element-group index e8 = (row * D + col) / 8 addresses
// x, residual, residual_out, norm_out (u32x4 = 8 bf16) and q (u32x2 = 8 codes)
// alike.
struct KArgs {
  const u32x4* x;
  const u32x4* res;
  const u32x4* gamma;
  u32x4* res_out;
  u32x4* norm_out;     // nullptr: 3-output form
  u32x2* q;
  void* scale;         // float* (SF_F32) or uint8_t* (SF_UE8M0)
  int64_t M;
  int32_t D;
  int32_t groups;      // D / G
  float eps;
  int32_t wpr;         // waves per row
  int32_t rpb;         // rows per workgroup
  int32_t col_major;   // scale layout: 0 -> [M, groups], 1 -> [groups, M]
  int32_t remap;       // 1 -> XCD-aware workgroup -> row-tile remap
};

// ---------------------------------------------------------------- helpers

__device__ __forceinline__ float bf16_lo(uint32_t v) { return __uint_as_float(v << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t v) { return __uint_as_float(v & 0xffff0000u); }

// Two fp32 -> packed bf16x2, round to nearest even (v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  typedef float f32x2 __attribute__((ext_vector_type(2)));
  typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
  f32x2 v = {lo, hi};
  bf16x2 b = __builtin_convertvector(v, bf16x2);
  return __builtin_bit_cast(uint32_t, b);
}

template <int CTRL>
__device__ __forceinline__ uint32_t umax_dpp(uint32_t m) {
  const uint32_t o = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)m, CTRL, 0xf, 0xf, false);
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
    const uint32_t o = (uint32_t)__shfl_xor((int)m, 16);
    m = m > o ? m : o;
  }
  return m;
}

__device__ __forceinline__ double wave_sum(double v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off);
  return v;
}

// Blocks are dispatched round-robin over the 8 XCDs (block b -> XCD b % 8).
// Give the blocks of one XCD consecutive row tiles so that neighbouring
// rows' column-major scale words meet in the same L2.
__device__ __forceinline__ int xcd_remap(int b, int nb) {
  const int x = b & 7, i = b >> 3, per = nb >> 3, rem = nb & 7;
  return x * per + (x < rem ? x : rem) + i;
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

// ---------------------------------------------------------------- kernel

template <int NS, int LPG, int QF, int SF>
__global__ void __launch_bounds__(NS <= 4 ? 1024 : 256)
fagq_rows(const KArgs a) {
  constexpr float QMAX = (QF == QF_FP8) ? 448.0f : 127.0f;
  constexpr int G = LPG * 8;
  __shared__ double s_part[kMaxWavesPerBlock];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wpr = a.wpr;
  const int blk = a.remap ? xcd_remap(blockIdx.x, gridDim.x) : (int)blockIdx.x;
  const int rib = wave / wpr;               // row within the workgroup
  const int part = wave - rib * wpr;        // wave within the row
  const int64_t row = (int64_t)blk * a.rpb + rib;
  const int D = a.D;
  const int c0 = part * (NS * kStepCols);   // first column of this wave
  const int rem_cols = (row < a.M) ? D - c0 : 0;
  // Steps entirely inside the row, and steps with at least one valid lane.
  const int nfull = rem_cols <= 0 ? 0 : (rem_cols >> 9 < NS ? rem_cols >> 9 : NS);
  const int nvalid = rem_cols <= 0 ? 0 : ((rem_cols + kStepCols - 1) >> 9 < NS ? (rem_cols + kStepCols - 1) >> 9 : NS);
  const int64_t e8row = row * (int64_t)(D >> 3) + (c0 >> 3) + lane;   // e8 index of step 0
  const int g8 = (c0 >> 3) + lane;                                    // gamma u32x4 index

  // Phase 1: issue every load of this wave's slice of the row.
  u32x4 xv[NS], rv[NS];
#pragma unroll
  for (int k = 0; k < NS; ++k) {
    if (k < nfull) {
      xv[k] = __builtin_nontemporal_load(a.x + e8row + k * 64);
      rv[k] = __builtin_nontemporal_load(a.res + e8row + k * 64);
    } else if (k < nvalid) {
      xv[k] = (u32x4){0u, 0u, 0u, 0u};
      rv[k] = (u32x4){0u, 0u, 0u, 0u};
      if (c0 + k * kStepCols + lane * 8 < D) {
        xv[k] = __builtin_nontemporal_load(a.x + e8row + k * 64);
        rv[k] = __builtin_nontemporal_load(a.res + e8row + k * 64);
      }
    }
  }

  // Phase 2: r = x + residual, residual_out, sum of squares (fp64), w = r * gamma,
  // per-group max |w|.
  double ss = 0.0;
  float w[NS][8];
  uint32_t gmax[NS];
#pragma unroll
  for (int k = 0; k < NS; ++k) {
    if (k < nvalid) {
      const bool lane_ok = (k < nfull) || (c0 + k * kStepCols + lane * 8 < D);
      u32x4 gv = (u32x4){0u, 0u, 0u, 0u};
      if (lane_ok) gv = a.gamma[g8 + k * 64];
      float r[8];
      u32x4 ro;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        r[2 * j] = bf16_lo(xv[k][j]) + bf16_lo(rv[k][j]);
        r[2 * j + 1] = bf16_hi(xv[k][j]) + bf16_hi(rv[k][j]);
        ro[j] = pack_bf16x2(r[2 * j], r[2 * j + 1]);
      }
      if (lane_ok) __builtin_nontemporal_store(ro, a.res_out + e8row + k * 64);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const double rd = (double)r[j];
        ss = __builtin_fma(rd, rd, ss);   // r^2 is exact in fp64
      }
      float m = 0.0f;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        w[k][2 * j] = r[2 * j] * bf16_lo(gv[j]);
        w[k][2 * j + 1] = r[2 * j + 1] * bf16_hi(gv[j]);
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) m = __builtin_fmaxf(m, __builtin_fabsf(w[k][j]));
      gmax[k] = group_max_bits<LPG>(__float_as_uint(m));
    }
  }

  // Phase 3: row sum of squares -> inv_rms.
  ss = wave_sum(ss);
  if (wpr > 1) {
    if (lane == 0) s_part[wave] = ss;
    __syncthreads();
    ss = 0.0;
    for (int p = 0; p < wpr; ++p) ss += s_part[rib * wpr + p];
  }
  const float sumsq = (float)ss;
  const float mean = sumsq / (float)D;
  const float inv = (float)(1.0 / __builtin_sqrt((double)(mean + a.eps)));
  const float inv_q = inv / QMAX;

  // Phase 4: scales, codes, optional norm_out.
#pragma unroll
  for (int k = 0; k < NS; ++k) {
    if (k < nvalid) {
      const int col = c0 + k * kStepCols + lane * 8;
      const bool lane_ok = (k < nfull) || (col < D);
      const float s = __builtin_fmaxf(__uint_as_float(gmax[k]) * inv_q, 1.0e-12f);
      float mul = 0.0f;
      int e = 0;
      if constexpr (SF == SF_F32) {
        mul = 1.0f / s;
      } else {
        e = ceil_log2_bits(s);
        e = e > 127 ? 127 : e;
      }
      float n[8], t[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        n[j] = w[k][j] * inv;
        const float u = (SF == SF_F32) ? n[j] * mul : __builtin_ldexpf(n[j], -e);
        t[j] = __builtin_fminf(__builtin_fmaxf(u, -QMAX), QMAX);
      }
      if (a.norm_out != nullptr) {
        u32x4 no;
#pragma unroll
        for (int j = 0; j < 4; ++j) no[j] = pack_bf16x2(n[2 * j], n[2 * j + 1]);
        if (lane_ok) __builtin_nontemporal_store(no, a.norm_out + e8row + k * 64);
      }
      const u32x2 codes = encode8<QF>(t);
      if (lane_ok) {
        __builtin_nontemporal_store(codes, a.q + e8row + k * 64);
        if ((lane & (LPG - 1)) == 0) {
          const int g = col / G;
          const int64_t si = a.col_major ? (int64_t)g * a.M + row : row * (int64_t)a.groups + g;
          if constexpr (SF == SF_F32) {
            static_cast<float*>(a.scale)[si] = s;
          } else {
            static_cast<uint8_t*>(a.scale)[si] = (uint8_t)(e + 127);
          }
        }
      }
    }
  }
}

// ---------------------------------------------------------------- diagnostics

// Encodes already-scaled fp32 values with the same device encoder as the
// operator (after the same clamp), 8 per thread.  n % 8 == 0.
template <int QF>
__global__ void __launch_bounds__(256) fagq_encode(const float* __restrict__ in,
                                                   u32x2* __restrict__ out, int64_t n8) {
  constexpr float QMAX = (QF == QF_FP8) ? 448.0f : 127.0f;
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n8) return;
  float t[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) t[j] = __builtin_fminf(__builtin_fmaxf(in[i * 8 + j], -QMAX), QMAX);
  out[i] = encode8<QF>(t);
}

}  // namespace fagq
