// mla_bwd.hip - gfx950 MLA backward (NoPE, shared K = V = C): dQ and dC as
// the reference's Task 03 operator computes them (C ABI: include/fagq_mla.h).
//
// Function (reference: src/task03_mla_bwd_nope_dkdv.py:401-425, :453-480):
//   rows i < E = min(16, S) of every (b, h): exact dq_i = sum_j dS_ij c_j with
//     P_ij = bf16(exp2((q_i . c_j * scale - lse_i) * log2 e)), j <= i,
//     dS_ij = bf16(P_ij (do_i . c_j - delta_i) scale), delta_i = out_i . do_i
//   rows i >= E: dq_i = scale * do_i
//   dc_j = sum_{i >= j} hs_i / (i + 1), hs_i = sum_h do[h, i]
//
// Kernels, in stream order:
//   K1 mla_stream_do   - the one pass over dO (all the HBM traffic): per row
//                        and all H heads, dq = scale * do (rows >= E) and the
//                        head sum, stored as hs_i / (i + 1) in the workspace.
//                        A lane owns 8 consecutive dims (16-byte loads), a
//                        workgroup 2048 / D rows, so each head contributes a
//                        contiguous 4 KB (D = 512) segment per workgroup.
//                        Short sequences split the heads into up to 8 groups,
//                        each writing a partial head-sum plane.
//   K2 mla_block_totals - per block of 16-64 rows (or column slice of one):
//                        fp32 totals of hs / (i + 1) over rows and head-group
//                        planes; each row's plane sum is written back over
//                        plane 0.
//   K3 mla_exact_rows_suffix_scan - one launch of 1024-thread workgroups, two
//                        kinds:
//                        * exact rows, one per (b, h): q, do and c rows 0..E-1
//                          in LDS, the logits and dP by bf16 MFMAs with fp32
//                          accumulation (one wave), P and dS rounded to bf16
//                          where the reference rounds, dq rows 0..E-1 (which
//                          K1 does not write);
//                        * per block: carry = totals of all later blocks, then
//                          the reverse running sum over the block's rows
//                          (plane 0), written as dc.
//                        The exact rows depend on nothing K1 or K2 writes;
//                        sharing the last launch with the few scan workgroups
//                        runs them in the part of the chip those leave idle.
// K2 and K3 issue each thread's loads as one batch: at these sizes they are
// latency-bound: every dependent round trip to memory adds its full latency.
//
// D above kSliceD (512) runs as column slices of at most kSliceD dims: K1, the
// block totals and K3 are per column, so each slice runs them on its columns
// (the tensors' row stride stays D, the workspace holds one slice), and the
// exact rows, whose dot products span all of D, run once over all columns in
// the first slice's K3, staging the rows in chunks of kSliceD dims.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <atomic>
#include <mutex>

#include "fagq.h"
#include "fagq_dispatch.hpp"
#include "fagq_mla.h"

namespace fagq {
namespace mla {
namespace {

constexpr int kThreads = 256;
constexpr int kE = FAGQ_MLA_EXACT_ROWS;
constexpr int kSliceD = FAGQ_MLA_SLICE_D;   // dims per column slice
constexpr int kPadElems = 8;             // LDS row padding (bf16 elements), exact rows
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

struct MArgs {
  const uint16_t* q;
  const uint16_t* c;
  const uint16_t* out;
  const uint16_t* dout;
  const float* lse;
  void* dq;
  void* dc;
  float* hs;          // workspace: [hsplit, B, S, D] partial head sums / (i + 1)
  float* tot;         // workspace: [B, nblk, D] block totals
  int64_t hs_split;   // elements between the partial head-sum planes (B * S * D)
  int32_t brows;      // rows per scan block
  int32_t nblk;       // ceil(S / brows)
  int32_t hsplit;     // head groups K1 splits the heads into
  int32_t hps;        // heads per group
  int32_t H, S;
  int32_t D;          // dims of this column slice (the width K1, K2 and K3's scan handle)
  int32_t ld;         // elements between rows of q, c, out, dout, dq and dc (the full D);
                      // their pointers point at the slice's first column
  int32_t nexact;     // K3 workgroups (x < nexact) running exact rows: H in the first slice
  int32_t erows;      // min(16, S)
  float scale;
  int32_t dq_bf16;    // dq is bf16 (else fp32)
  int32_t dc_bf16;
  int32_t bsplit_sh;  // K2 workgroups per scan block = 1 << bsplit_sh, each summing
                      // D >> bsplit_sh of its columns
};

__device__ __forceinline__ float bf16_to_f(uint32_t h) { return __uint_as_float(h << 16); }

// fp32 -> bf16 bits, round to nearest even (v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint32_t f_to_bf16(float v) { return pack_bf16x2(v, 0.0f) & 0xffffu; }
__device__ __forceinline__ float round_bf16(float v) { return bf16_to_f(f_to_bf16(v)); }

// Stores 8 fp32 values at element offset e of an fp32 or bf16 tensor.
__device__ __forceinline__ void store8(const rsrc_t& rs, bool bf16, uint32_t e, const float (&v)[8]) {
  if (bf16) {
    const u32x4 w = {pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]), pack_bf16x2(v[4], v[5]),
                     pack_bf16x2(v[6], v[7])};
    __builtin_amdgcn_raw_buffer_store_b128(w, rs, e * 2u, 0, kNonTemporal);
  } else {
    const u32x4 a = {__float_as_uint(v[0]), __float_as_uint(v[1]), __float_as_uint(v[2]),
                     __float_as_uint(v[3])};
    const u32x4 b = {__float_as_uint(v[4]), __float_as_uint(v[5]), __float_as_uint(v[6]),
                     __float_as_uint(v[7])};
    __builtin_amdgcn_raw_buffer_store_b128(a, rs, e * 4u, 0, kNonTemporal);
    __builtin_amdgcn_raw_buffer_store_b128(b, rs, e * 4u + 16u, 0, kNonTemporal);
  }
}

// ------------------------------------------------------------------ K1

// grid (ceil(S / rows_per_wg), B, hsplit); rows_per_wg = 256 / (D / 8);
// z picks the head group [z hps, min(H, (z + 1) hps)).  U heads' loads are in
// flight per lane: for grids of 2048 and more U = 2 with bf16 dq (50 VGPRs, 8
// workgroups per CU) and U = 1 with fp32 dq, whose stores are twice the
// loads' bytes (2 B / 4 B, 2 x 64 x 4096 x 512: 297 against 308 us for the
// pass); U = 8 (110 VGPRs, 4 per CU) for grids that fit 4 per CU, where each
// workgroup's few heads are then loaded at once.
template <int U, bool HALVES>
__global__ void __launch_bounds__(kThreads) mla_stream_do(const MArgs g) {
  const int lpr = g.D / 8;                        // lanes per row
  const int t = threadIdx.x;
  // When lpr does not divide kThreads, the last kThreads % lpr threads hold
  // no whole row of this workgroup (their t / lpr would be the next
  // workgroup's first row), and stop here.
  if (t / lpr >= kThreads / lpr) return;
  const int row = (int)blockIdx.x * (kThreads / lpr) + t / lpr;
  if (row >= g.S) return;
  const int b = (int)blockIdx.y;
  const int hbeg = (int)blockIdx.z * g.hps;
  const int hend = hbeg + g.hps < g.H ? hbeg + g.hps : g.H;
  const uint32_t hsd = (uint32_t)g.H * (uint32_t)g.S * (uint32_t)g.ld;   // elements per batch
  // The slice's elements of batch b end at (H S - 1) ld + D (the descriptors'
  // size, so they stay inside the tensors whatever the slice's first column).
  const uint32_t span = hsd - (uint32_t)g.ld + (uint32_t)g.D;
  const rsrc_t rdo = make_rsrc(g.dout + (int64_t)b * hsd, span * 2u);
  const rsrc_t rdq = make_rsrc((const uint8_t*)g.dq + (int64_t)b * hsd * (g.dq_bf16 ? 2 : 4),
                               span * (g.dq_bf16 ? 2u : 4u));
  // Elements of the lane (head 0): 8 consecutive from ea, or with HALVES 4
  // from ea and 4 from eb = ea + D / 2, so that each of its two 16-byte fp32
  // stores lies in a contiguous half-row span of the row's lanes.  wa / wb:
  // the same elements in the workspace's head-sum plane, rows of D.
  const uint32_t li = (uint32_t)(t % lpr);
  const uint32_t lo = li * (HALVES ? 4u : 8u);
  const uint32_t ea = (uint32_t)row * (uint32_t)g.ld + lo;
  const uint32_t eb = ea + (uint32_t)g.D / 2u;
  const uint32_t wa = (uint32_t)row * (uint32_t)g.D + lo;
  const uint32_t wb = wa + (uint32_t)g.D / 2u;
  const uint32_t hstride = (uint32_t)g.S * (uint32_t)g.ld;
  const bool write_dq = row >= g.erows;
  const bool dq_bf16 = g.dq_bf16 != 0;
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  // Heads in batches of U, software-pipelined: the loads of batch i + 1 are
  // issued before batch i is consumed.  Heads past hend re-read head hend - 1
  // (in bounds) and are not used.
  auto load_batch = [&](int h0, u32x4 (&v)[U]) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int h = h0 + u < hend ? h0 + u : hend - 1;
      const uint32_t ho = (uint32_t)h * hstride;
      if constexpr (HALVES) {
        const u32x2 x = __builtin_amdgcn_raw_buffer_load_b64(rdo, (ea + ho) * 2u, 0, kNonTemporal);
        const u32x2 y = __builtin_amdgcn_raw_buffer_load_b64(rdo, (eb + ho) * 2u, 0, kNonTemporal);
        v[u] = u32x4{x[0], x[1], y[0], y[1]};
      } else {
        v[u] = __builtin_amdgcn_raw_buffer_load_b128(rdo, (ea + ho) * 2u, 0, kNonTemporal);
      }
    }
  };
  // 8 fp32 values of the lane: one 16-byte bf16 or two 16-byte fp32 stores at
  // element xa (HALVES: the second at xb).
  auto store_lane = [&](const rsrc_t& rs, bool bf16, uint32_t xa, uint32_t xb, const float (&v)[8]) {
    if constexpr (HALVES) {
      const u32x4 x = {__float_as_uint(v[0]), __float_as_uint(v[1]), __float_as_uint(v[2]),
                       __float_as_uint(v[3])};
      const u32x4 y = {__float_as_uint(v[4]), __float_as_uint(v[5]), __float_as_uint(v[6]),
                       __float_as_uint(v[7])};
      __builtin_amdgcn_raw_buffer_store_b128(x, rs, xa * 4u, 0, kNonTemporal);
      __builtin_amdgcn_raw_buffer_store_b128(y, rs, xb * 4u, 0, kNonTemporal);
    } else {
      store8(rs, bf16, xa, v);
    }
  };
  u32x4 cur[U], nxt[U];
  load_batch(hbeg, cur);
  for (int h0 = hbeg; h0 < hend; h0 += U) {
    if (h0 + U < hend) load_batch(h0 + U, nxt);
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (h0 + u < hend) {
        float f[8];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          f[2 * k] = bf16_lo(cur[u][k]);
          f[2 * k + 1] = bf16_hi(cur[u][k]);
        }
#pragma unroll
        for (int k = 0; k < 8; ++k) acc[k] += f[k];
        if (write_dq) {
          float d[8];
#pragma unroll
          for (int k = 0; k < 8; ++k) d[k] = f[k] * g.scale;
          const uint32_t ho = (uint32_t)(h0 + u) * hstride;
          store_lane(rdq, dq_bf16, ea + ho, eb + ho, d);
        }
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) cur[u] = nxt[u];
  }
  const float n1 = (float)(row + 1);
  float o[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) o[k] = acc[k] / n1;
  const uint32_t sd = (uint32_t)g.S * (uint32_t)g.D;
  const rsrc_t rhs = make_rsrc(g.hs + (int64_t)blockIdx.z * g.hs_split + (int64_t)b * sd, sd * 4u);
  store_lane(rhs, false, wa, wb, o);
}

// ------------------------------------------------------------------ K3: exact rows

constexpr int kWide = 1024;               // threads of K2 and K3 (16 waves)

// Exact rows 0..E-1 of (b, h), wave m owning query row m for delta and dq;
// wave 0 computes all 16 x 16 logits and dP with MFMAs.  The rows' D = ld
// dims go through LDS in chunks of W = min(D, kSliceD): per chunk, every
// global load is issued before the first LDS store (wave m loads 16-byte
// piece `lane` of its q, do and out rows, thread t piece t % (W / 8) of c
// row t / (W / 8)); buffer descriptors over rows 0..E-1 return zeros for the
// rest.  The logits, dP and delta accumulate over the chunks; dS follows; then
// dq, chunk by chunk (c staged again when D > W).  Dynamic LDS: q, do and c
// rows 0..15 of one chunk (padded by 16 bytes), then dS [16][16] and delta [16].
__device__ __forceinline__ void exact_rows(const MArgs& g, int b, int h) {
  extern __shared__ __align__(16) uint8_t smem[];
  const int D = g.ld, E = g.erows;
  const int W = D < kSliceD ? D : kSliceD;
  const int ldl = W + kPadElems;                  // bf16 elements per LDS row
  uint16_t* qs = reinterpret_cast<uint16_t*>(smem);
  uint16_t* dos = qs + kE * ldl;
  uint16_t* cs = dos + kE * ldl;
  float* dS = reinterpret_cast<float*>(cs + kE * ldl);
  float* deltas = dS + kE * kE;                   // [kE], after dS
  const int t = threadIdx.x, lane = t & 63, m = t >> 6;
  const int bh = b * g.H + h;
  const int64_t qrow0 = (int64_t)bh * g.S * D;    // q, do, out rows of (b, h)
  const uint32_t rbytes = (uint32_t)(E * D * 2);
  const rsrc_t rq = make_rsrc(g.q + qrow0, rbytes);
  const rsrc_t rdo = make_rsrc(g.dout + qrow0, rbytes);
  const rsrc_t rout = make_rsrc(g.out + qrow0, rbytes);
  const rsrc_t rc = make_rsrc(g.c + (int64_t)b * g.S * D, rbytes);
  // c rows 0..15 of the W-wide chunk at dim c0 (t < 16 W / 8 <= 1024).
  auto stage_c = [&](int c0, int cpr) {
    const int cr = t / cpr;
    const uint32_t coff = cr < E ? (uint32_t)(cr * D + c0 + (t % cpr) * 8) * 2u : rbytes;
    const u32x4 cv = __builtin_amdgcn_raw_buffer_load_b128(rc, coff, 0, 0);
    if (t < kE * cpr) *reinterpret_cast<u32x4*>(cs + cr * ldl + (t % cpr) * 8) = cv;
  };

  // Logits and dP of query row qm = lane % 16 with keys n = 4 (lane / 16) +
  // r (r < 4), by wave 0 alone: v_mfma_f32_16x16x32_bf16 with A = c rows
  // (key), B = q or dO rows (query), K = the chunk's dims in steps of 32.
  // Lane l supplies row l % 16 of both operands, 8 consecutive dims (the same
  // ones for both) per step, and receives D[4 (l / 16) + r][l % 16] (checked
  // on the GPU).  Rows past E were staged as zeros.
  const int qm = lane & 15, k0 = (lane >> 4) * 8;
  f32x4 lg = {0.0f, 0.0f, 0.0f, 0.0f}, dpv = lg;
  float delta = 0.0f;
  for (int c0 = 0; c0 < D; c0 += W) {
    const int w = D - c0 < W ? D - c0 : W;        // a multiple of 64
    const int cpr = w / 8;                        // 16-byte pieces per row (8..64)
    if (c0 > 0) __syncthreads();                  // the previous chunk's reads are done
    const uint32_t off = m < E && lane < cpr ? (uint32_t)(m * D + c0 + lane * 8) * 2u : rbytes;
    const u32x4 a = __builtin_amdgcn_raw_buffer_load_b128(rq, off, 0, 0);
    const u32x4 d = __builtin_amdgcn_raw_buffer_load_b128(rdo, off, 0, 0);
    const u32x4 o = __builtin_amdgcn_raw_buffer_load_b128(rout, off, 0, 0);
    stage_c(c0, cpr);
    if (lane < cpr) {
      *reinterpret_cast<u32x4*>(qs + m * ldl + lane * 8) = a;
      *reinterpret_cast<u32x4*>(dos + m * ldl + lane * 8) = d;
    }
    // delta_m = out_m . do_m, this lane's part.
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      delta += bf16_lo(o[j]) * bf16_lo(d[j]);
      delta += bf16_hi(o[j]) * bf16_hi(d[j]);
    }
    __syncthreads();
    if (m == 0) {
      const uint16_t* cr = cs + qm * ldl + k0;
      const uint16_t* qr = qs + qm * ldl + k0;
      const uint16_t* dr = dos + qm * ldl + k0;
      auto ld8 = [](const uint16_t* p) { return *reinterpret_cast<const bf16x8*>(p); };
#pragma unroll 2
      for (int k = 0; k < w; k += 64) {           // w % 64 == 0: two steps per pass
        const bf16x8 c0v = ld8(cr + k), q0 = ld8(qr + k), d0 = ld8(dr + k);
        const bf16x8 c1v = ld8(cr + k + 32), q1 = ld8(qr + k + 32), d1 = ld8(dr + k + 32);
        lg = __builtin_amdgcn_mfma_f32_16x16x32_bf16(c0v, q0, lg, 0, 0, 0);
        dpv = __builtin_amdgcn_mfma_f32_16x16x32_bf16(c0v, d0, dpv, 0, 0, 0);
        lg = __builtin_amdgcn_mfma_f32_16x16x32_bf16(c1v, q1, lg, 0, 0, 0);
        dpv = __builtin_amdgcn_mfma_f32_16x16x32_bf16(c1v, d1, dpv, 0, 0, 0);
      }
    }
  }
#pragma unroll
  for (int s = 32; s > 0; s >>= 1) delta += __shfl_xor(delta, s, 64);
  if (lane == 0) deltas[m] = delta;
  __syncthreads();
  if (m == 0) {
    const float lse = qm < E ? g.lse[(int64_t)bh * g.S + qm] : 0.0f;
    const float dlt = deltas[qm];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int kn = 4 * (lane >> 4) + r;
      float sv = 0.0f;
      if (qm < E && kn <= qm) {
        const float p = round_bf16(exp2f((lg[r] * g.scale - lse) * 1.4426950408889634f));
        sv = round_bf16(p * (dpv[r] - dlt) * g.scale);
      }
      dS[qm * kE + kn] = sv;
    }
  }
  __syncthreads();

  // dq row m, chunk by chunk: lane owns dims c0 + 8 lane .. + 7.
  const rsrc_t rdq = make_rsrc((const uint8_t*)g.dq + qrow0 * (g.dq_bf16 ? 2 : 4),
                               (uint32_t)(E * D) * (g.dq_bf16 ? 2u : 4u));
  for (int c0 = 0; c0 < D; c0 += W) {
    const int w = D - c0 < W ? D - c0 : W;
    if (D > W) {                                  // c of this chunk (one chunk: still staged)
      __syncthreads();
      stage_c(c0, w / 8);
      __syncthreads();
    }
    if (m < E && lane * 8 < w) {
      const int k = lane * 8;
      float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
      for (int j = 0; j <= m; ++j) {
        const float sv = dS[m * kE + j];
        const u32x4 c = *reinterpret_cast<const u32x4*>(cs + j * ldl + k);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          acc[2 * i] = fmaf(sv, bf16_lo(c[i]), acc[2 * i]);
          acc[2 * i + 1] = fmaf(sv, bf16_hi(c[i]), acc[2 * i + 1]);
        }
      }
      store8(rdq, g.dq_bf16 != 0, (uint32_t)(m * D + c0 + k), acc);
    }
  }
}

// Dynamic LDS of K3: the exact rows' rows and dS.
size_t exact_lds_bytes(int64_t D) {
  const int64_t W = D < kSliceD ? D : kSliceD;
  return (size_t)3 * kE * (W + kPadElems) * 2 + (size_t)(kE * kE + kE) * 4;
}
constexpr size_t kBlockTotalLds = (size_t)kWide * 16;   // dynamic LDS of K2: the parts' join

// ------------------------------------------------------------------ K2: block totals

constexpr int kBatch = 16;                // loads issued before they are used

__device__ __forceinline__ void add4(float4& a, const float4& b) {
  a.x += b.x;
  a.y += b.y;
  a.z += b.z;
  a.w += b.w;
}

// Thread layout of K2's block totals and K3 over D columns (K2: the
// workgroup's column slice): cpt = D / 4 column threads (16..128) per part,
// np = kWide / cpt parts (8..64); thread t owns columns 4 (t % cpt) .. + 3 of
// part t / cpt (threads of parts >= np idle).
struct Parts {
  int cpt, np, p, col;
  __device__ explicit Parts(int D) : cpt(D >> 2), np(kWide / (D >> 2)), p((int)threadIdx.x / (D >> 2)),
                                     col((int)threadIdx.x - p * (D >> 2)) {}
};

// Part p of the block's threads sums rows r0 + p, r0 + p + np, ... of the
// block over the HS head-group planes; a batch loads all planes of
// kBatch / HS such rows together.  With HS > 1 each row's plane sum
// (planes in order) is written back over plane 0, so K3 reads one plane.
// The parts' totals are joined in LDS, in part order.
template <int HS>
__device__ __forceinline__ void block_total_hs(const MArgs& g, int b, int blk, int cs, float4* part) {
  constexpr int R = kBatch / HS;
  const int cols = g.D >> g.bsplit_sh;            // this workgroup's columns: cs cols .. + cols
  const Parts P(cols);
  const int r0 = blk * g.brows;
  const int r1 = r0 + g.brows < g.S ? r0 + g.brows : g.S;
  float* __restrict__ hs = g.hs + (int64_t)b * g.S * g.D + cs * cols + 4 * P.col;
  float4 a = make_float4(0.f, 0.f, 0.f, 0.f);
  if (P.p < P.np) {
    for (int r = r0 + P.p; r < r1; r += R * P.np) {
      float4 v[R][HS];
#pragma unroll
      for (int i = 0; i < R; ++i) {
        const int rr = r + i * P.np < r1 ? r + i * P.np : r0;
#pragma unroll
        for (int s = 0; s < HS; ++s)
          v[i][s] = *reinterpret_cast<const float4*>(hs + s * g.hs_split + (int64_t)rr * g.D);
      }
#pragma unroll
      for (int i = 0; i < R; ++i) {
        const int rr = r + i * P.np;
        if (rr < r1) {
          float4 sum = v[i][0];
#pragma unroll
          for (int s = 1; s < HS; ++s) add4(sum, v[i][s]);
          if (HS > 1) *reinterpret_cast<float4*>(hs + (int64_t)rr * g.D) = sum;
          add4(a, sum);
        }
      }
    }
  }
  part[threadIdx.x] = a;
  __syncthreads();
  if (P.p == 0) {
    for (int q = 1; q < P.np; ++q) add4(a, part[q * P.cpt + P.col]);
    *reinterpret_cast<float4*>(g.tot + ((int64_t)b * g.nblk + blk) * g.D + cs * cols + 4 * P.col) = a;
  }
}

// Totals of block blk (g.brows rows) of batch b over rows and head groups,
// columns of slice cs (D >> bsplit_sh wide).
__device__ __forceinline__ void block_total(const MArgs& g, int b, int blk, int cs) {
  extern __shared__ __align__(16) uint8_t smem[];
  float4* part = reinterpret_cast<float4*>(smem);
  switch (g.hsplit) {                     // 1..8 (kMaxHeadSplit)
    case 1: block_total_hs<1>(g, b, blk, cs, part); break;
    case 2: block_total_hs<2>(g, b, blk, cs, part); break;
    case 3: block_total_hs<3>(g, b, blk, cs, part); break;
    case 4: block_total_hs<4>(g, b, blk, cs, part); break;
    case 5: block_total_hs<5>(g, b, blk, cs, part); break;
    case 6: block_total_hs<6>(g, b, blk, cs, part); break;
    case 7: block_total_hs<7>(g, b, blk, cs, part); break;
    default: block_total_hs<8>(g, b, blk, cs, part); break;
  }
}

// grid (nblk << bsplit_sh, B): 1 << bsplit_sh workgroups per block.
__global__ void __launch_bounds__(kWide) mla_block_totals(const MArgs g) {
  const int x = (int)blockIdx.x, b = (int)blockIdx.y;
  block_total(g, b, x >> g.bsplit_sh, x & ((1 << g.bsplit_sh) - 1));
}

// ------------------------------------------------------------------ K3

constexpr int kChunkRows = 8;             // >= ceil(64 / 8): rows per part of a block

// Block blk of batch b.  The block's rows are np chunks of cr = ceil(brows /
// np) rows (cr <= 8 since brows <= 64 and np >= 8); part p scans chunk p.
// Part p first sums (1) the totals of later blocks blk + 1 + p, blk + 1 + p +
// np, ... and (2) the rows of its chunk (kept in registers); after one
// barrier its carry is all parts' (1), in part order, plus the (2) of the
// chunks above it, then the reverse running sum over the chunk is written as
// dc.
__device__ __forceinline__ void suffix_scan(const MArgs& g, int b, int blk) {
  __shared__ float4 later[kWide], chunk[kWide];
  const Parts P(g.D);
  const int r0 = blk * g.brows;
  const int r1 = r0 + g.brows < g.S ? r0 + g.brows : g.S;
  const int cr = (g.brows + P.np - 1) / P.np;
  const int c0 = r0 + P.p * cr < r1 ? r0 + P.p * cr : r1;
  const int c1 = c0 + cr < r1 ? c0 + cr : r1;
  // The workspace and dc never overlap (checked at launch): restrict lets the
  // loads issue together ahead of the stores.
  const float* __restrict__ hs = g.hs + (int64_t)b * g.S * g.D + 4 * P.col;
  const float* __restrict__ tot = g.tot + (int64_t)b * g.nblk * g.D + 4 * P.col;
  float4 rows[kChunkRows];
  float4 lat = make_float4(0.f, 0.f, 0.f, 0.f), own = lat;
  if (P.p < P.np) {
#pragma unroll
    for (int k = 0; k < kChunkRows; ++k)        // rows c1 - 1 - k (clamped)
      rows[k] = *reinterpret_cast<const float4*>(hs + (int64_t)(c1 - 1 - k >= c0 ? c1 - 1 - k : r0) * g.D);
    for (int x = blk + 1 + P.p; x < g.nblk; x += kBatch * P.np) {
      float4 v[kBatch];
#pragma unroll
      for (int k = 0; k < kBatch; ++k) {
        const int xx = x + k * P.np;
        v[k] = *reinterpret_cast<const float4*>(tot + (int64_t)(xx < g.nblk ? xx : x) * g.D);
      }
#pragma unroll
      for (int k = 0; k < kBatch; ++k)
        if (x + k * P.np < g.nblk) add4(lat, v[k]);
    }
#pragma unroll
    for (int k = 0; k < kChunkRows; ++k)
      if (c1 - 1 - k >= c0) add4(own, rows[k]);
  }
  later[threadIdx.x] = lat;
  chunk[threadIdx.x] = own;
  __syncthreads();
  if (P.p >= P.np || c0 >= c1) return;
  float4 cy = make_float4(0.f, 0.f, 0.f, 0.f);
  for (int q = 0; q < P.np; ++q) add4(cy, later[q * P.cpt + P.col]);
  for (int q = P.np - 1; q > P.p; --q) add4(cy, chunk[q * P.cpt + P.col]);
  float* __restrict__ dcf = static_cast<float*>(g.dc) + (int64_t)b * g.S * g.ld + 4 * P.col;
  uint16_t* __restrict__ dch = static_cast<uint16_t*>(g.dc) + (int64_t)b * g.S * g.ld + 4 * P.col;
  const bool bf16 = g.dc_bf16 != 0;
#pragma unroll
  for (int k = 0; k < kChunkRows; ++k) {
    const int r = c1 - 1 - k;
    if (r >= c0) {
      add4(cy, rows[k]);
      if (bf16) {
        const uint2 wv = {pack_bf16x2(cy.x, cy.y), pack_bf16x2(cy.z, cy.w)};
        *reinterpret_cast<uint2*>(dch + (int64_t)r * g.ld) = wv;
      } else {
        *reinterpret_cast<float4*>(dcf + (int64_t)r * g.ld) = cy;
      }
    }
  }
}

// grid (nexact + nblk, B): x < nexact (H in the first column slice, else 0)
// are the exact rows of head x, the rest the scan of block x - nexact.
// Uniform per workgroup, so every barrier sees all its waves.
__global__ void __launch_bounds__(kWide) mla_exact_rows_suffix_scan(const MArgs g) {
  const int x = (int)blockIdx.x, b = (int)blockIdx.y;
  if (x < g.nexact)
    exact_rows(g, b, x);
  else
    suffix_scan(g, b, x - g.nexact);
}

bool aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }

bool overlap(const void* a, int64_t na, const void* b, int64_t nb) {
  const uintptr_t x = reinterpret_cast<uintptr_t>(a), y = reinterpret_cast<uintptr_t>(b);
  return na > 0 && nb > 0 && x < y + (uintptr_t)nb && y < x + (uintptr_t)na;
}

constexpr int kMinK1Groups = 1024;        // K1 workgroups wanted (4 per CU)
constexpr int64_t kCUs = 256;             // compute units of an MI355X
constexpr int kMaxHeadSplit = 8;

// Head groups for K1 when the row grid alone is small: doubles while the grid
// has fewer than kMinK1Groups workgroups (at most 8 groups, never more than H).
int64_t head_split(int64_t B, int64_t S, int64_t D, int64_t H) {
  if (D < 64) return 1;
  const int64_t rows_per_wg = kThreads / (D / 8);
  const int64_t base = ((S + rows_per_wg - 1) / rows_per_wg) * B;
  int64_t sp = 1;
  while (base * sp < kMinK1Groups && sp < kMaxHeadSplit && sp * 2 <= H) sp *= 2;
  return sp;
}

// Workgroups per scan block for the block totals.  Short sequences, where K1
// splits the heads into several partial head-sum planes, leave few blocks
// whose workgroups each read brows rows of every plane (and write the plane
// sums back); from 128 KB per workgroup that read sets K2's length, and the
// block is split into up to 4 column slices of at least 128 dims while K2's
// grid (B nblk split workgroups) stays within one per CU.  Measured (B 2, H
// 64, D 512): S 256 and 512 split 4 ways, 3-5 % faster per call; a split of
// the single-plane S 4096 blocks (128 KB, 128 workgroups) 1 % slower.
int32_t block_split(int64_t B, int64_t nblk, int64_t brows, int64_t hsplit, int64_t ds) {
  if (hsplit < 2 || brows * hsplit * ds * 4 < (128 << 10)) return 1;
  int32_t sp = 1;
  while (sp < 4 && ds % (2 * sp * 64) == 0 && ds / (2 * sp) >= 128 && B * nblk * 2 * sp <= kCUs)
    sp *= 2;
  return sp;
}

// Rows per scan block: S / 64 rounded up to a multiple of 16, within [16, 64],
// so short sequences still spread over many blocks and each thread's carry and
// in-block loops stay short.
int64_t block_rows(int64_t S) {
  int64_t r = ((S + 63) / 64 + 15) / 16 * 16;
  return r < 16 ? 16 : r > 64 ? 64 : r;
}

// Dims of column slice `i` of D (slices of kSliceD, the last one shorter).
int64_t slice_dims(int64_t D, int64_t i) {
  const int64_t rest = D - i * kSliceD;
  return rest < kSliceD ? rest : kSliceD;
}

// The workspace holds one column slice at a time: the most any of D's slices
// (kSliceD wide, the last one D % kSliceD when that is not 0) needs.
int64_t workspace_bytes(int64_t B, int64_t S, int64_t D) {
  if (B < 0 || S < 0 || D < 0 || B > (1 << 20) || S > (1ll << 31) || D > (1ll << 31)) return -1;
  const int64_t nblk = (S + block_rows(S) - 1) / block_rows(S);
  auto slice_bytes = [&](int64_t w) {
    const int64_t sp = head_split(B, S, w, kMaxHeadSplit);   // the most any H can use
    return (sp * B * S + B * nblk) * w * 4;
  };
  const int64_t a = slice_bytes(D < kSliceD ? D : kSliceD);
  const int64_t b = D > kSliceD && D % kSliceD ? slice_bytes(D % kSliceD) : 0;
  return a > b ? a : b;
}

}  // namespace
}  // namespace mla
}  // namespace fagq

using namespace fagq;
using namespace fagq::mla;

extern "C" {

FAGQ_API int64_t fagq_mla_bwd_workspace_bytes(int64_t B, int64_t S, int64_t D) {
  return workspace_bytes(B, S, D);
}

}  // extern "C"

namespace fagq {
namespace mla {
namespace {

// Argument checks shared by both entry points (everything but the workspace);
// *need receives the workspace bytes the call uses.
int check_args(const void* q, const void* c_kv, const void* out, const void* dout,
               const float* lse, void* dq, void* dc_kv, int64_t B, int64_t H, int64_t S,
               int64_t D, float sm_scale, int dq_dtype, int dc_dtype, int64_t* need) {
  if (!q || !c_kv || !out || !dout || !lse || !dq || !dc_kv) return FAGQ_E_NULL;
  if ((dq_dtype != FAGQ_MLA_F32 && dq_dtype != FAGQ_MLA_BF16) ||
      (dc_dtype != FAGQ_MLA_F32 && dc_dtype != FAGQ_MLA_BF16))
    return FAGQ_E_FORMAT;
  if (B < 0 || H < 1 || S < 1 || D < 64 || D % 64 != 0 || !(sm_scale == sm_scale))
    return FAGQ_E_SHAPE;
  if (B > 65535 || H > 65535 || H * S * D * 4 >= (1ll << 32)) return FAGQ_E_TOO_LARGE;
  *need = workspace_bytes(B, S, D);
  if (*need < 0) return FAGQ_E_TOO_LARGE;
  if (!aligned(q, 16) || !aligned(c_kv, 16) || !aligned(out, 16) || !aligned(dout, 16) ||
      !aligned(lse, 4) || !aligned(dq, 16) || !aligned(dc_kv, 16))
    return FAGQ_E_ALIGN;
  return FAGQ_OK;
}

// Overlap checks with the workspace, the device check and the three launches.
int launch(const void* q, const void* c_kv, const void* out, const void* dout, const float* lse,
           void* dq, void* dc_kv, void* workspace, int64_t need, int64_t B, int64_t H, int64_t S,
           int64_t D, float sm_scale, int dq_dtype, int dc_dtype, void* stream) {
  const int64_t nq = B * H * S * D * 2, nc = B * S * D * 2, nl = B * H * S * 4;
  const int64_t ndq = B * H * S * D * (dq_dtype == FAGQ_MLA_BF16 ? 2 : 4);
  const int64_t ndc = B * S * D * (dc_dtype == FAGQ_MLA_BF16 ? 2 : 4);
  const void* ins[5] = {q, c_kv, out, dout, lse};
  const int64_t nin[5] = {nq, nc, nq, nq, nl};
  void* outs[3] = {dq, dc_kv, workspace};
  const int64_t nout[3] = {ndq, ndc, need};
  for (int i = 0; i < 3; ++i) {
    for (int j = 0; j < 5; ++j)
      if (overlap(outs[i], nout[i], ins[j], nin[j])) return FAGQ_E_ALIAS;
    for (int j = i + 1; j < 3; ++j)
      if (overlap(outs[i], nout[i], outs[j], nout[j])) return FAGQ_E_ALIAS;
  }
  const int dcheck = device_check();
  if (dcheck != FAGQ_OK) return dcheck;

  // One pass per column slice; every slice's kernels run in stream order, so
  // each reuses the workspace after the previous slice's K3 has read it.
  const int64_t nslice = (D + kSliceD - 1) / kSliceD;
  const int64_t qb = dq_dtype == FAGQ_MLA_BF16 ? 2 : 4, cb = dc_dtype == FAGQ_MLA_BF16 ? 2 : 4;
  hipStream_t st = static_cast<hipStream_t>(stream);
  for (int64_t sl = 0; sl < nslice; ++sl) {
    const int64_t col = sl * kSliceD, ds = slice_dims(D, sl);
    MArgs g;
    g.q = static_cast<const uint16_t*>(q);         // the exact rows (first slice) read all of D
    g.c = static_cast<const uint16_t*>(c_kv);
    g.out = static_cast<const uint16_t*>(out);
    g.dout = static_cast<const uint16_t*>(dout) + col;
    g.lse = lse;
    g.dq = static_cast<uint8_t*>(dq) + col * qb;   // K1's rows; the exact rows run with col = 0
    g.dc = static_cast<uint8_t*>(dc_kv) + col * cb;
    const int64_t hsplit = head_split(B, S, ds, H);
    g.hps = (int32_t)((H + hsplit - 1) / hsplit);
    g.hsplit = (int32_t)((H + g.hps - 1) / g.hps);        // non-empty head groups
    g.hs = static_cast<float*>(workspace);
    g.hs_split = B * S * ds;
    g.brows = (int32_t)block_rows(S);
    g.nblk = (int32_t)((S + g.brows - 1) / g.brows);
    g.tot = g.hs + g.hsplit * B * S * ds;
    g.H = (int32_t)H;
    g.S = (int32_t)S;
    g.D = (int32_t)ds;
    g.ld = (int32_t)D;
    g.nexact = sl == 0 ? (int32_t)H : 0;
    const int32_t bsplit = block_split(B, g.nblk, g.brows, g.hsplit, ds);
    g.bsplit_sh = bsplit == 4 ? 2 : bsplit == 2 ? 1 : 0;
    g.erows = (int32_t)(S < kE ? S : kE);
    g.scale = sm_scale;
    g.dq_bf16 = dq_dtype == FAGQ_MLA_BF16;
    g.dc_bf16 = dc_dtype == FAGQ_MLA_BF16;
    void* args[] = {&g};
    const int rows_per_wg = kThreads / (int)(ds / 8);
    const dim3 k1_grid((unsigned)((S + rows_per_wg - 1) / rows_per_wg), (unsigned)B,
                       (unsigned)g.hsplit);
    const bool k1_wide = (int64_t)k1_grid.x * k1_grid.y * k1_grid.z <= kMinK1Groups;
    const bool halves = dq_dtype == FAGQ_MLA_F32;
    const void* k1 = halves ? (k1_wide ? reinterpret_cast<const void*>(&mla_stream_do<8, true>)
                                       : reinterpret_cast<const void*>(&mla_stream_do<1, true>))
                            : (k1_wide ? reinterpret_cast<const void*>(&mla_stream_do<8, false>)
                                       : reinterpret_cast<const void*>(&mla_stream_do<2, false>));
    int ls = launch_kernel(k1, k1_grid, dim3(kThreads), args, 0, st);
    if (ls != FAGQ_OK) return ls;
    // 4 nblk < 2^22 and nexact + nblk < 2^17 + 2^20: nblk <= S / 16 + 1 and
    // H S D 4 < 2^32 with D >= 64.
    ls = launch_kernel(reinterpret_cast<const void*>(&mla_block_totals),
                       dim3((unsigned)(g.nblk * bsplit), (unsigned)B), dim3(kWide), args,
                       kBlockTotalLds, st);
    if (ls != FAGQ_OK) return ls;
    ls = launch_kernel(reinterpret_cast<const void*>(&mla_exact_rows_suffix_scan),
                       dim3((unsigned)(g.nexact + g.nblk), (unsigned)B), dim3(kWide), args,
                       g.nexact ? exact_lds_bytes(D) : 0, st);
    if (ls != FAGQ_OK) return ls;
  }
  return FAGQ_OK;
}

// The workspace of fagq_mla_bwd_launch_noalloc: one array per GPU the library
// runs on, held until the process ends.  Host code never passes `scratch`
// itself to a kernel (in host code the name is a stand-in, not the device
// address): the device address is looked up once per device, with that
// device current, and used instead.
static __device__ __align__(256) uint8_t scratch[FAGQ_MLA_SCRATCH_BYTES];

constexpr int kMaxScratchDevices = 64;
std::atomic<void*> g_scratch_addr[kMaxScratchDevices];
std::mutex g_scratch_mu;

// Device address of the current device's `scratch`; FAGQ_OK or an error.
int scratch_address(void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return -(int)e;
  if (dev < 0 || dev >= kMaxScratchDevices) return FAGQ_E_DEVICE;
  void* p = g_scratch_addr[dev].load(std::memory_order_acquire);
  if (!p) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    p = g_scratch_addr[dev].load(std::memory_order_relaxed);
    if (!p) {
      e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
      if (e != hipSuccess) return -(int)e;
      if (!p) return FAGQ_E_DEVICE;
      g_scratch_addr[dev].store(p, std::memory_order_release);
    }
  }
  *out = p;
  return FAGQ_OK;
}

}  // namespace
}  // namespace mla
}  // namespace fagq

extern "C" {

FAGQ_API int fagq_mla_bwd_launch(const void* q, const void* c_kv, const void* out, const void* dout,
                                 const float* lse, void* dq, void* dc_kv, void* workspace,
                                 int64_t ws_bytes, int64_t B, int64_t H, int64_t S, int64_t D,
                                 float sm_scale, int dq_dtype, int dc_dtype, void* stream) {
  int64_t need = 0;
  const int v = check_args(q, c_kv, out, dout, lse, dq, dc_kv, B, H, S, D, sm_scale, dq_dtype,
                           dc_dtype, &need);
  if (v != FAGQ_OK) return v;
  if (!workspace) return FAGQ_E_NULL;
  if (ws_bytes < need) return FAGQ_E_SHAPE;
  if (!aligned(workspace, 16)) return FAGQ_E_ALIGN;
  if (B == 0) return FAGQ_OK;
  return launch(q, c_kv, out, dout, lse, dq, dc_kv, workspace, need, B, H, S, D, sm_scale,
                dq_dtype, dc_dtype, stream);
}

FAGQ_API int fagq_mla_bwd_launch_noalloc(const void* q, const void* c_kv, const void* out,
                                         const void* dout, const float* lse, void* dq,
                                         void* dc_kv, int64_t B, int64_t H, int64_t S, int64_t D,
                                         float sm_scale, int dq_dtype, int dc_dtype, void* stream) {
  int64_t need = 0;
  const int v = check_args(q, c_kv, out, dout, lse, dq, dc_kv, B, H, S, D, sm_scale, dq_dtype,
                           dc_dtype, &need);
  if (v != FAGQ_OK) return v;
  if (need > FAGQ_MLA_SCRATCH_BYTES) return FAGQ_E_TOO_LARGE;
  if (B == 0) return FAGQ_OK;
  const int dcheck = device_check();
  if (dcheck != FAGQ_OK) return dcheck;
  void* ws = nullptr;
  const int sa = scratch_address(&ws);
  if (sa != FAGQ_OK) return sa;
  return launch(q, c_kv, out, dout, lse, dq, dc_kv, ws, need, B, H, S, D, sm_scale, dq_dtype,
                dc_dtype, stream);
}

}  // extern "C"
