// fagq_gemm.hip - gfx950 fp8 block-scaled GEMM that consumes the quantizer's
// codes and per-token 1 x 128 scales (C ABI: include/fagq_gemm.h).
//
//   C[m, n] = bf16( sum_kb fp32(sa(m, kb) * sb(n / 128, kb)) * P_kb[m, n] )
//
// No counterpart in the reference repository (its operator,
// src/task01_fused_add_rmsnorm_group_quant.py:1731-1851, stops at the
// quantized tensor and scales); this is the layer those formats feed.
//
// Work mapping.  A workgroup computes a 256 x BN tile of C (BN = 256, or 192
// where that suits N): 8 waves of 64 x BN / 2 for every scale format, each
// wave a grid of 16 x 16 tiles, each one v_mfma_scale_f32_16x16x128_f8f6f4
// per 128-deep k-block.  The weight tile is the MFMA's first operand and the activation
// tile its second, so each lane's four results are four consecutive columns
// of one row of C (lane l: row l % 16, columns 4 (l / 16) .. +4) and the
// activation scale a lane needs is that of its own row.
//
// Operand staging.  Per k-block, the 256 x 128- and BN x 128-byte tiles of A and B go from
// global memory straight into LDS (buffer_load_dwordx4 ... lds: each
// instruction writes 1 KB, 16 bytes per lane, in lane order).  LDS holds
// each 128-byte row with its eight 16-byte chunks XOR-swizzled: logical chunk
// c of row r sits at position c ^ f(r), f(r) = ((r >> 1) & 1) | ((r & 4) ? 4 : 0),
// so a lane fetches the logical chunk (lane % 8) ^ f(r).  An MFMA operand read
// is 16 consecutive rows at one logical chunk per 16 lanes.  gfx950 serves a
// ds_read_b128 in four passes of 16 lanes over the 64 banks (4 cycles when no
// two lanes of a pass hit one bank at different addresses); the lanes of a
// pass are not 16 consecutive ones.  fagq_diag_lds_read (include/fagq_diag.h)
// measures the fragment read with this f at 4 cycles per instruction and with
// f(r) = (r >> 1) & 7 or r & 7 at 8 (a 2-way conflict on every read).
//
// Pipeline (fagq_gemm_pp_kernel).  Five 32 KB slots, all 160 KB of LDS,
// hold the tile sequence A(0), B(0), A(1), B(1), ...; the 8 waves are two
// groups of four half a k-block apart, so that one group's products run
// while the other reads its fragments from LDS and issues the copies.
//
// Scales.  fp32 (or mixed) scales: each k-block's 16 x 16 x 128 product goes
// to a temporary and is added to the accumulator as t * (sa * sb) with fmaf.
// Both UE8M0: the matrix core applies 2^(ea - 127) and 2^(eb - 127) itself
// (the MFMA's per-lane E8M0 operands), which is exact, so the product
// accumulates directly.
//
// Every global access goes through a buffer descriptor sized to the
// workgroup's rows: rows of A or B past M or N read zeros and stores of rows
// past M are dropped in hardware; column tiles past N are skipped (N % 16 ==
// 0, so a 16-column tile is wholly inside or outside).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "fagq.h"
#include "fagq_diag.h"
#include "fagq_dispatch.hpp"
#include "fagq_gemm.h"
#include "fagq_gemm_lds.hpp"

namespace fagq {
namespace gemm {
namespace {

typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void_t;

constexpr int kBM = 256;                 // rows of C per workgroup
constexpr int kMaxBN = 256;              // columns of C per workgroup, at most
constexpr int kATileBytes = kBM * kBK;   // the activation tile of one stage in LDS
constexpr int kGroupM = 4;               // row tiles per group of the tile order
constexpr int kCUs = 256;                // compute units of a gfx950 MI355X / MI350X

// Wave layouts of the 256 x BN tile.  WAVES_M x WAVES_N waves, each owning
// TM x TN tiles of 16 x 16.  8 waves of 64 x (BN / 2) for every format: with
// two waves per SIMD one wave's MFMAs cover the other's LDS reads.  (4 waves
// of 128 x 128, accumulators in AGPRs, read a third less from LDS per MFMA
// but measured 15 % slower with UE8M0 scales: one wave per SIMD leaves the
// operand reads after each barrier exposed.)  BN is 256, or 192 where that
// tiles N into fewer column-weighted rounds of the CUs (N = 2112: 11 tiles
// of 192 against 9 of 256, the last a quarter full).  A wave's columns then
// start at a multiple of 96 and may span two 128-column weight blocks.
template <int BN_, int WAVES_M_, int WAVES_N_>
struct Layout {
  static constexpr int BN = BN_;
  static constexpr int WAVES_M = WAVES_M_, WAVES_N = WAVES_N_;
  static constexpr int WAVES = WAVES_M * WAVES_N;
  static constexpr int THREADS = 64 * WAVES;
  static constexpr int TM = kBM / 16 / WAVES_M;
  static constexpr int TN = BN / 16 / WAVES_N;
  static constexpr int B_TILE_BYTES = BN * kBK;
  // A wave's columns lie in one weight block unless they can straddle two.
  static constexpr bool SPLIT = BN % 128 != 0 || (16 * TN) % 128 != 0;
  static_assert(16 * TN <= 128, "a wave's columns touch at most two 128-column weight blocks");
  static_assert(BN <= kMaxBN, "tile width");
};
using Layout256 = Layout<256, 4, 2>;
using Layout192 = Layout<192, 4, 2>;
constexpr int kVmcnt0 = 0x0F70;          // s_waitcnt vmcnt(0) (other counters not waited)
// s_waitcnt vmcnt(n), other counters not waited (n < 64).
constexpr int vmcnt_imm(int n) { return (n & 15) | ((n >> 4) << 14) | 0x0F70; }
constexpr int kSlotBytes = kATileBytes;  // ring slot: one operand tile
constexpr int kSlots = 5;                // 160 KB, all of a gfx950 CU's LDS
static_assert(kMaxBN * kBK <= kSlotBytes, "a weight tile fits a ring slot");

struct GArgs {
  const uint8_t* a;       // fp8 [M, K]
  const uint8_t* as;      // activation scales
  const uint8_t* b;       // fp8 [N, K]
  const uint8_t* bs;      // weight scales [ceil(N / 128), K / 128]
  uint16_t* c;            // bf16 [M, N]
  int32_t M, N, K;
  int32_t kblocks;        // K / 128
  int32_t as_kstride;     // elements between the scales of consecutive k-blocks of one row
  int32_t as_mstride;     // elements between the scales of consecutive rows
  int32_t m_tiles, n_tiles;
  uint32_t as_bytes, bs_bytes;
};

// Workgroup b runs on XCD b % 8.  XCD x takes one contiguous range of the
// tile order, and the order walks kGroupM row tiles at a time column by
// column, so the tiles an XCD has in flight share a few row and column
// panels in its L2.
__device__ __forceinline__ void tile_coords(int b, int m_tiles, int n_tiles, int& mt, int& nt) {
  const int T = m_tiles * n_tiles;
  const int x = b & 7, i = b >> 3, per = T >> 3, rem = T & 7;
  const int t = x * per + (x < rem ? x : rem) + i;
  const int group = t / (kGroupM * n_tiles);
  const int first_m = group * kGroupM;
  const int gm = m_tiles - first_m < kGroupM ? m_tiles - first_m : kGroupM;
  const int w = t - group * kGroupM * n_tiles;
  mt = first_m + w % gm;
  nt = w / gm;
}


// One 16 x 128-byte MFMA operand: lane l gets row (r0 + l % 16), k bytes
// 32 (l / 16) .. +32, from a swizzled LDS tile.
__device__ __forceinline__ i32x8 lds_frag(const uint8_t* tile, int row, int lane) {
  const int c0 = (lane >> 4) * 2;
  const int sw = swz_of(row);
  const uint8_t* r = tile + row * kBK;
  const i32x4 lo = *reinterpret_cast<const i32x4*>(r + ((c0 ^ sw) << 4));
  const i32x4 hi = *reinterpret_cast<const i32x4*>(r + (((c0 + 1) ^ sw) << 4));
  return i32x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
}

__device__ __forceinline__ float e8m0_to_f32(uint32_t e) {
  // 2^(e - 127); e = 0 is the subnormal 2^-127 (e = 255, NaN, never produced).
  return e ? __uint_as_float(e << 23) : __uint_as_float(0x00400000u);
}

// Keeps the memory instructions on either side in issue order.
__device__ __forceinline__ void issue_order_fence() { asm volatile("" ::: "memory"); }
// Workgroup barrier once this wave's LDS reads have returned; the caller has
// waited for whichever LDS copies must have landed (__syncthreads would also
// wait for every copy still in flight).
__device__ __forceinline__ void ring_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}
// The value is computed before this point, in program order with the other
// volatile asm statements (the compiler would otherwise sink MFMAs, which
// have no memory operands, past a wait and barrier).
__device__ __forceinline__ void pin(const f32x4& v) { asm volatile("" ::"v"(v)); }

// ring_barrier() fenced for the scheduler as well: nothing moves across it,
// so the products of a product interval cannot be hoisted into the read
// interval before it (MFMAs have no memory operands, and the compiler
// otherwise interleaves them with the fragment reads).
__device__ __forceinline__ void pp_barrier() {
  __builtin_amdgcn_sched_barrier(0);
  ring_barrier();
  __builtin_amdgcn_sched_barrier(0);
}

// The GEMM kernel: the ping-pong pipeline.  The 8 waves form two groups of
// 4: group 0 (waves 0-3) owns the tile's columns 0 .. BN / 2 - 1, group 1
// (waves 4-7) the other half, and each SIMD runs one wave of each.  Every
// k-block spans two barrier intervals, and group 1 runs half a k-block
// behind group 0, so in each interval one group reads its operand fragments
// from LDS (and issues copies) while the other runs its 32 products from
// registers:
//   interval 2k + 1: group 0 reads k-block k's fragments  | group 1 multiplies k - 1
//   interval 2k + 2: group 0 multiplies k                  | group 1 reads k
// A wave holds a whole k-block's fragments (4 activation and BN / 32 weight
// 16 x 128-byte operands) between its read and product intervals.  Five 32 KB
// LDS slots form a ring over the tile sequence A(0), B(0), A(1), B(1), ...
// (A(k) in slot 2k % 5, B(k) in 2k + 1 % 5):
// group 0 copies B(k + 1) while reading k, group 1 copies A(k + 2) while
// reading k, and each waits for its own copies before the barrier that ends
// its next product interval (B) or read interval (A), so every copy has one
// k-block to land.  A copy only fills a slot whose last reader finished
// before the barrier that precedes the copy.  Both groups run the same
// number of iterations and barriers; past the last k-block group 1 still
// multiplies once, and group 0 waits at the barriers.
template <int ASF, int BSF, class L>
__global__ void __launch_bounds__(L::THREADS, 1) fagq_gemm_pp_kernel(const GArgs g) {
  static_assert(L::WAVES_M == 4 && L::WAVES_N == 2, "two groups of four 64 x BN / 2 waves");
  constexpr bool kHwScale = ASF == SF_UE8M0 && BSF == SF_UE8M0;
  constexpr int kTM = L::TM, kTN = L::TN;
  constexpr int kNB = L::SPLIT ? 2 : 1;            // weight blocks a wave's columns touch
  // 1 KB copies per wave: group 1 copies the activation tile, group 0 the weight tile.
  constexpr int kCopyA = kATileBytes / 1024 / 4, kCopyB = L::B_TILE_BYTES / 1024 / 4;
  static_assert(kCopyA * 4096 == kATileBytes && kCopyB * 4096 == L::B_TILE_BYTES,
                "four waves copy each tile");
  constexpr int kScaleLoads = kTM + kNB;           // memory instructions of load_scales
  // At BN = 192 the reading group runs at raised wave priority during its
  // reads and copies (q_a + kv_a 256.7 -> 241.7 us, same box); at BN = 256 that
  // measured 0.8-1 % slower.
  constexpr bool kReadPrio = L::BN != 256;
  __shared__ __attribute__((aligned(1024))) uint8_t lds[kSlots * kSlotBytes];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave % L::WAVES_M, wn = wave / L::WAVES_M;
  const bool g0 = wn == 0;
  int mt, nt;
  tile_coords((int)blockIdx.x, g.m_tiles, g.n_tiles, mt, nt);
  const int m0 = mt * kBM, n0 = nt * L::BN;
  const int mrows = g.M - m0 < kBM ? g.M - m0 : kBM;
  const int nrows = g.N - n0 < L::BN ? g.N - n0 : L::BN;
  const rsrc_t ra = make_rsrc(g.a + (int64_t)m0 * g.K, (uint32_t)mrows * (uint32_t)g.K);
  const rsrc_t rb = make_rsrc(g.b + (int64_t)n0 * g.K, (uint32_t)nrows * (uint32_t)g.K);
  const rsrc_t ras = make_rsrc(g.as, g.as_bytes);
  const rsrc_t rbs = make_rsrc(g.bs, g.bs_bytes);

  // Copy geometry: the four waves of a group copy one whole tile; copy
  // instruction u of wave wm is instruction i = wm C + u of the tile (C =
  // kCopyA or kCopyB) and fills LDS rows 8 i .. +8.  The lane's row within
  // them is lane / 8, its position lane % 8, and it fetches the logical chunk
  // stored there; the swizzle of row 8 i + lane / 8 depends on lane / 8
  // only, so one lane offset serves every instruction.  The whole offset goes
  // in the VGPR offset and the scalar offset is zero: the hardware
  // range-checks only the VGPR offset (plus the immediate), so this is what
  // turns rows past M or N into zero reads.  Offsets are computed in uint32:
  // the launch checks that every one fits.
  const int crow = lane >> 3;
  const uint32_t cvoff = (uint32_t)crow * (uint32_t)g.K + (uint32_t)swz(lane & 7, crow) * 16u;
  auto copy_one = [&](const rsrc_t& rs, int kb, uint8_t* dst, int inst) {
    const uint32_t off = cvoff + (uint32_t)__builtin_amdgcn_readfirstlane(
        (int)((uint32_t)inst * 8u * (uint32_t)g.K + (uint32_t)kb * (uint32_t)kBK));
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void_t*)(dst + inst * 1024), 16, off, 0, 0, 0);
  };
  auto issue_a = [&](int kb, int slot) {
#pragma unroll
    for (int u = 0; u < kCopyA; ++u) copy_one(ra, kb, lds + slot * kSlotBytes, wm * kCopyA + u);
  };
  auto issue_b = [&](int kb, int slot) {
#pragma unroll
    for (int u = 0; u < kCopyB; ++u) copy_one(rb, kb, lds + slot * kSlotBytes, wm * kCopyB + u);
  };

  // Scale bits of the lane's rows (m0 + 16 (TM wm + i) + lane % 16) and of
  // the 128-column weight blocks of the wave's columns (block wblk for tiles
  // j < jsplit, wblk + 1 for the rest), as loaded bits.  Offsets as for the
  // copies: all in the range-checked VGPR offset, so scale reads for rows
  // past M or weight blocks past N read zeros (those rows and columns are
  // never stored).
  const int arow = m0 + wm * 16 * kTM + (lane & 15);
  const int wcol = n0 + wn * 16 * kTN;
  const int wblk = wcol >> 7;
  const int jsplit = L::SPLIT ? (((wblk + 1) << 7) - wcol) >> 4 : kTN;
  constexpr uint32_t asb = ASF == SF_F32 ? 4u : 1u, bsb = BSF == SF_F32 ? 4u : 1u;
  const uint32_t a_voff = (uint32_t)arow * (uint32_t)g.as_mstride * asb;
  struct Scales {
    uint32_t a[kTM], b[kNB];
  };
  auto load_scales = [&](int kb) {
    Scales sc;
#pragma unroll
    for (int h = 0; h < kNB; ++h) {
      const uint32_t boff = (uint32_t)__builtin_amdgcn_readfirstlane(
          (int)(((uint32_t)(wblk + h) * (uint32_t)g.kblocks + (uint32_t)kb) * bsb));
      sc.b[h] = BSF == SF_F32 ? __builtin_amdgcn_raw_buffer_load_b32(rbs, boff, 0, 0)
                              : (uint32_t)__builtin_amdgcn_raw_buffer_load_b8(rbs, boff, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < kTM; ++i) {
      const uint32_t e = (uint32_t)kb * (uint32_t)g.as_kstride +
                         16u * (uint32_t)i * (uint32_t)g.as_mstride;
      const uint32_t off = a_voff + (uint32_t)__builtin_amdgcn_readfirstlane((int)(e * asb));
      sc.a[i] = ASF == SF_F32 ? __builtin_amdgcn_raw_buffer_load_b32(ras, off, 0, 0)
                              : (uint32_t)__builtin_amdgcn_raw_buffer_load_b8(ras, off, 0, 0);
    }
    return sc;
  };

  f32x4 acc[kTN][kTM];
#pragma unroll
  for (int j = 0; j < kTN; ++j)
#pragma unroll
    for (int i = 0; i < kTM; ++i) acc[j][i] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  i32x8 af[kTM], bf[kTN];
  auto read_frags = [&](int kb) {
    const int sa = (2 * kb) % kSlots, sb = (2 * kb + 1) % kSlots;
    const uint8_t* ta = lds + sa * kSlotBytes;
    const uint8_t* tb = lds + sb * kSlotBytes;
#pragma unroll
    for (int i = 0; i < kTM; ++i) af[i] = lds_frag(ta, wm * 16 * kTM + 16 * i + (lane & 15), lane);
#pragma unroll
    for (int j = 0; j < kTN; ++j) bf[j] = lds_frag(tb, wn * 16 * kTN + 16 * j + (lane & 15), lane);
  };
  // One k-block's products.  Both UE8M0: the matrix core applies the scales.
  // fp32 (or mixed): each product goes to a temporary and is added as
  // fmaf(t, sa * sb, acc), and the schedule
  // alternates one MFMA with four FMAs, so that a product's promotion runs
  // while the next MFMA executes.
  auto products = [&](const Scales& s) {
    if constexpr (kHwScale) {
#pragma unroll
      for (int j = 0; j < kTN; ++j) {
        const int sbj = (int)(L::SPLIT && j >= jsplit ? s.b[kNB - 1] : s.b[0]);
#pragma unroll
        for (int i = 0; i < kTM; ++i)
          acc[j][i] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
              bf[j], af[i], acc[j][i], 0, 0, 0, sbj, 0, (int)s.a[i]);
      }
    } else {
      float sm[kNB][kTM];
#pragma unroll
      for (int h = 0; h < kNB; ++h) {
        const float sb = BSF == SF_UE8M0 ? e8m0_to_f32(s.b[h]) : __uint_as_float(s.b[h]);
#pragma unroll
        for (int i = 0; i < kTM; ++i)
          sm[h][i] = (ASF == SF_UE8M0 ? e8m0_to_f32(s.a[i]) : __uint_as_float(s.a[i])) * sb;
      }
#pragma unroll
      for (int j = 0; j < kTN; ++j) {
        const bool hi = L::SPLIT && j >= jsplit;   // weight block wblk + 1; uniform over the wave
#pragma unroll
        for (int i = 0; i < kTM; ++i) {
          const float smv = hi ? sm[kNB - 1][i] : sm[0][i];
          const f32x4 t = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
              bf[j], af[i], f32x4{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0, 127, 0, 127);
#pragma unroll
          for (int r = 0; r < 4; ++r) acc[j][i][r] = __builtin_fmaf(t[r], smv, acc[j][i][r]);
        }
      }
#pragma unroll
      for (int n = 0; n < kTN * kTM; ++n) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // one MFMA
        __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);   // four VALU
      }
    }
#pragma unroll
    for (int j = 0; j < kTN; ++j)
#pragma unroll
      for (int i = 0; i < kTM; ++i) pin(acc[j][i]);
  };

  const int nk = g.kblocks, last = nk - 1;
  // Past the last k-block the copies and scale loads fetch the last k-block
  // again, into the slots the next k-blocks would take (free at that point,
  // and never read): every iteration issues the same instructions, so the
  // in-order counter's waits are constants (a scale wait does not also wait
  // for the copies issued after the scales).
  // Each group runs its own loop (the branch is uniform per wave); both pass
  // 2 nk + 2 barriers, so every barrier is met by all 8 waves.  Barrier
  // 2k + 2 starts group 0's products of k-block k and group 1's reads of it;
  // barrier 2k + 3 starts group 1's products of k and group 0's reads of k + 1.
  if (g0) {
    // Prologue: A(0); with group 1's B(0) it lands before the first barrier.
    issue_a(0, 0);
    __builtin_amdgcn_s_waitcnt(kVmcnt0);
    pp_barrier();
#pragma clang loop unroll(disable)
    for (int k = 0; k < nk; ++k) {
      // Reads k-block k and copies B(k + 1) into the slot A(k - 1) left.
      if constexpr (kReadPrio) __builtin_amdgcn_s_setprio(1);
      const Scales cur = load_scales(k);
      issue_order_fence();
      read_frags(k);
      issue_order_fence();
      issue_b(k + 1 < last ? k + 1 : last, (2 * k + 3) % kSlots);
      if constexpr (kReadPrio) __builtin_amdgcn_s_setprio(0);
      pp_barrier();
      // Multiplies k while group 1 reads it.
      products(cur);
      __builtin_amdgcn_s_waitcnt(kVmcnt0);   // B(k + 1) has landed
      pp_barrier();
    }
    pp_barrier();                           // while group 1 multiplies the last k-block
  } else {
    // Prologue: B(0), then A(1) left in flight.
    issue_b(0, 1);
    issue_order_fence();
    issue_a(1 < last ? 1 : last, 2);
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(kCopyA));
    pp_barrier();
    pp_barrier();                           // group 0 reads k-block 0
    Scales cur;
#pragma clang loop unroll(disable)
    for (int k = 0; k < nk; ++k) {
      // Reads k-block k (group 0 multiplies it) and copies A(k + 2) into
      // the slot B(k - 1) left; A(k + 1) must land before the barrier.
      if constexpr (kReadPrio) __builtin_amdgcn_s_setprio(1);
      cur = load_scales(k);                   // first: the products wait for them at the barrier
      issue_order_fence();
      read_frags(k);
      issue_order_fence();
      issue_a(k + 2 < last ? k + 2 : last, (2 * k + 4) % kSlots);
      if constexpr (kReadPrio) __builtin_amdgcn_s_setprio(0);
      __builtin_amdgcn_s_waitcnt(vmcnt_imm(kScaleLoads + kCopyA));
      pp_barrier();
      // Multiplies k while group 0 reads k + 1.
      products(cur);
      pp_barrier();
    }
  }
  __builtin_amdgcn_s_waitcnt(kVmcnt0);

  const rsrc_t rc = make_rsrc(g.c + (int64_t)m0 * g.N, (uint32_t)mrows * (uint32_t)g.N * 2u);
#pragma unroll
  for (int j = 0; j < kTN; ++j) {
    const int ncol = wcol + 16 * j;
    if (ncol >= g.N) continue;   // uniform over the wave
#pragma unroll
    for (int i = 0; i < kTM; ++i) {
      const uint32_t row = (uint32_t)(wm * 16 * kTM + 16 * i + (lane & 15));
      u32x2 v;
      v[0] = pack_bf16x2(acc[j][i][0], acc[j][i][1]);
      v[1] = pack_bf16x2(acc[j][i][2], acc[j][i][3]);
      const uint32_t off = (row * (uint32_t)g.N + (uint32_t)(ncol + 4 * (lane >> 4))) * 2u;
      __builtin_amdgcn_raw_buffer_store_b64(v, rc, off, 0, 0);
    }
  }
}

bool aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }

int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

bool overlap(const void* a, int64_t na, const void* b, int64_t nb) {
  const uintptr_t a0 = reinterpret_cast<uintptr_t>(a), b0 = reinterpret_cast<uintptr_t>(b);
  return a0 < b0 + (uintptr_t)nb && b0 < a0 + (uintptr_t)na;
}

int validate(const void* a_q, const void* a_scale, const void* b_q, const void* b_scale,
             const void* c, int64_t M, int64_t N, int64_t K, int asf, int asl, int bsf) {
  if (!a_q || !a_scale || !b_q || !b_scale || !c) return FAGQ_E_NULL;
  if ((asf != FAGQ_SCALE_F32 && asf != FAGQ_SCALE_UE8M0) ||
      (bsf != FAGQ_SCALE_F32 && bsf != FAGQ_SCALE_UE8M0) ||
      (asl != FAGQ_LAYOUT_ROW_MAJOR && asl != FAGQ_LAYOUT_COL_MAJOR))
    return FAGQ_E_FORMAT;
  if (M < 0 || N <= 0 || K <= 0 || N % 16 != 0 || K % kBK != 0) return FAGQ_E_SHAPE;
  const int64_t kb = K / kBK;
  const int64_t asb = asf == FAGQ_SCALE_F32 ? 4 : 1, bsb = bsf == FAGQ_SCALE_F32 ? 4 : 1;
  // 32-bit buffer offsets: one workgroup's rows of A, B and C, and each scale array.
  if (M > INT32_MAX || (int64_t)kBM * K > (int64_t)UINT32_MAX ||
      (int64_t)kMaxBN * K > (int64_t)UINT32_MAX || (int64_t)kBM * N * 2 > (int64_t)UINT32_MAX ||
      M * kb * asb > (int64_t)UINT32_MAX || ceil_div(N, 128) * kb * bsb > (int64_t)UINT32_MAX ||
      ceil_div(M, kBM) * ceil_div(N, Layout192::BN) > INT32_MAX)
    return FAGQ_E_TOO_LARGE;
  if (!aligned(a_q, 16) || !aligned(b_q, 16) || !aligned(c, 16) ||
      (asf == FAGQ_SCALE_F32 && !aligned(a_scale, 4)) ||
      (bsf == FAGQ_SCALE_F32 && !aligned(b_scale, 4)))
    return FAGQ_E_ALIGN;
  if (M == 0) return FAGQ_OK;
  const int64_t cb = M * N * 2;
  if (overlap(c, cb, a_q, M * K) || overlap(c, cb, b_q, N * K) ||
      overlap(c, cb, a_scale, M * kb * asb) || overlap(c, cb, b_scale, ceil_div(N, 128) * kb * bsb))
    return FAGQ_E_ALIAS;
  return FAGQ_OK;
}

// Kernel for a pair of scale formats and a tile width.
template <class L>
const void* kernel_for_layout(int asf, int bsf) {
  const bool au = asf == FAGQ_SCALE_UE8M0, bu = bsf == FAGQ_SCALE_UE8M0;
  if (au && bu) return reinterpret_cast<const void*>(&fagq_gemm_pp_kernel<SF_UE8M0, SF_UE8M0, L>);
  if (au) return reinterpret_cast<const void*>(&fagq_gemm_pp_kernel<SF_UE8M0, SF_F32, L>);
  if (bu) return reinterpret_cast<const void*>(&fagq_gemm_pp_kernel<SF_F32, SF_UE8M0, L>);
  return reinterpret_cast<const void*>(&fagq_gemm_pp_kernel<SF_F32, SF_F32, L>);
}
static_assert(Layout256::THREADS == Layout192::THREADS, "one workgroup size");

// Tile width: 256 unless 192 takes fewer column-weighted rounds of the CUs
// (one workgroup per CU at a time), cost(BN) = ceil(tiles(BN) / CUs) * BN;
// ties keep 256.
int pick_bn(int64_t M, int64_t N) {
  auto cost = [&](int64_t bn) { return ceil_div(ceil_div(M, kBM) * ceil_div(N, bn), kCUs) * bn; };
  return cost(Layout192::BN) < cost(Layout256::BN) ? Layout192::BN : Layout256::BN;
}

int launch(const void* a_q, const void* a_scale, const void* b_q, const void* b_scale, void* c,
           int64_t M, int64_t N, int64_t K, int asf, int asl, int bsf, int bn, void* stream) {
  const int v = validate(a_q, a_scale, b_q, b_scale, c, M, N, K, asf, asl, bsf);
  if (v != FAGQ_OK || M == 0) return v;
  const int dc = device_check();
  if (dc != FAGQ_OK) return dc;
  if (bn == 0) bn = pick_bn(M, N);
  GArgs g;
  g.a = static_cast<const uint8_t*>(a_q);
  g.as = static_cast<const uint8_t*>(a_scale);
  g.b = static_cast<const uint8_t*>(b_q);
  g.bs = static_cast<const uint8_t*>(b_scale);
  g.c = static_cast<uint16_t*>(c);
  g.M = (int32_t)M;
  g.N = (int32_t)N;
  g.K = (int32_t)K;
  g.kblocks = (int32_t)(K / kBK);
  const bool col = asl == FAGQ_LAYOUT_COL_MAJOR;
  g.as_kstride = col ? (int32_t)M : 1;
  g.as_mstride = col ? 1 : g.kblocks;
  g.m_tiles = (int32_t)ceil_div(M, kBM);
  g.n_tiles = (int32_t)ceil_div(N, bn);
  g.as_bytes = (uint32_t)(M * g.kblocks * (asf == FAGQ_SCALE_F32 ? 4 : 1));
  g.bs_bytes = (uint32_t)(ceil_div(N, 128) * g.kblocks * (bsf == FAGQ_SCALE_F32 ? 4 : 1));
  void* args[] = {&g};
  const void* kernel = bn == Layout192::BN ? kernel_for_layout<Layout192>(asf, bsf)
                                           : kernel_for_layout<Layout256>(asf, bsf);
  return launch_kernel(kernel, dim3((unsigned)(g.m_tiles * g.n_tiles)),
                       dim3((unsigned)Layout256::THREADS), args, 0,
                       static_cast<hipStream_t>(stream));
}

}  // namespace
}  // namespace gemm
}  // namespace fagq

using namespace fagq;
using namespace fagq::gemm;

extern "C" {

FAGQ_API int fagq_gemm_launch(const void* a_q, const void* a_scale, const void* b_q,
                              const void* b_scale, void* c, int64_t M, int64_t N, int64_t K,
                              int a_scale_format, int a_scale_layout, int b_scale_format,
                              void* stream) {
  return launch(a_q, a_scale, b_q, b_scale, c, M, N, K, a_scale_format, a_scale_layout,
                b_scale_format, 0, stream);
}

FAGQ_API int fagq_gemm_launch_mapped(const void* a_q, const void* a_scale, const void* b_q,
                                     const void* b_scale, void* c, int64_t M, int64_t N,
                                     int64_t K, int a_scale_format, int a_scale_layout,
                                     int b_scale_format, int block_n, void* stream) {
  if (block_n != 0 && block_n != Layout192::BN && block_n != Layout256::BN) return FAGQ_E_FORMAT;
  return launch(a_q, a_scale, b_q, b_scale, c, M, N, K, a_scale_format, a_scale_layout,
                b_scale_format, block_n, stream);
}

FAGQ_API int fagq_gemm_query_route(int64_t M, int64_t N, int64_t K, fagq_gemm_route* route) {
  if (!route) return FAGQ_E_NULL;
  if (M < 0 || N <= 0 || K <= 0 || N % 16 != 0 || K % kBK != 0) return FAGQ_E_SHAPE;
  const int bn = pick_bn(M, N);
  route->block_m = kBM;
  route->block_n = bn;
  route->block_threads = Layout256::THREADS;
  route->group_m = kGroupM;
  route->grid_blocks = ceil_div(M, kBM) * ceil_div(N, bn);
  return FAGQ_OK;
}

}  // extern "C"
