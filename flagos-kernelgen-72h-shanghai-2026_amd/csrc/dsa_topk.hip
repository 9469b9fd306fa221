// dsa_topk.hip - gfx950 DSA top-k page-table transform (Task 02 of the
// reference repository), C ABI in include/fagq_dsa.h.
//
// Function (reference: src/task02_dsa_topk_page_table_transform.py:154-175
// and :1666; reports/task02_dsa_topk_page_table_transform.md:21-28): for
// every query row (b, h, q) of scores[B, H, Q, NB], the blocks of the causal
// valid prefix are ordered by score descending, then block id ascending,
// and the first top_k block ids and their page_table[b, id] entries are
// written (-1 past the number of selectable blocks).
//
// Work mapping.  One wave per row, four rows per workgroup.  A lane holds
// EPL scores of the row in VGPRs (NB <= 64 * EPL), loaded as 16-byte vectors
// through a buffer descriptor sized to the row's valid prefix: blocks past
// it are never fetched.
//
// Selection is exact and never sorts the whole row:
//   * Every selectable block has a 64-bit composite key, (ordered score bits
//     << 32) | (0xffffffff - id): larger is better, so the order is score
//     descending then id ascending, -0 and +0 mapped to one key.
//   * If at most CAP (512) blocks are selectable they are all candidates.
//   * Otherwise a 256-bin histogram in LDS, over the scores' fp32 range (the
//     bin is a monotone function of the score), locates the bin holding the
//     top_k-th block; the blocks above it are in the result and the bin is
//     the new search range, kept as [lo, hi] bounds on the composite key.
//     While more than CAP blocks lie at or above the range, the range is
//     split again by a 256-bin histogram on the composite key itself, which
//     always separates its smallest and largest keys, so the loop ends.
//   * The candidates (composite key >= lo, at most CAP) are compacted to
//     LDS, bitonic-sorted in registers across the wave (descending), and the
//     first top_k are written together with their page-table entries.
// For Gaussian-like scores the fp32 histogram leaves a handful of blocks in
// the boundary bin, so a row costs one histogram and a sort of about top_k
// keys.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "fagq.h"
#include "fagq_dispatch.hpp"
#include "fagq_dsa.h"

namespace fagq {
namespace dsa {
namespace {

constexpr int kRowsPerBlock = 4;
constexpr int kThreads = 64 * kRowsPerBlock;
constexpr int kBins = 256;
constexpr int kCap = 512;            // candidates sorted at most
constexpr int kMaxTopK = FAGQ_DSA_MAX_TOP_K;

struct DArgs {
  const void* scores;
  const int32_t* page_table;
  const void* q_pos;
  const void* kv_lens;
  int32_t* out_blocks;
  int32_t* out_pages;
  int64_t rows;          // B * H * Q
  int32_t H, Q, NB;
  int32_t block_size;
  int32_t top_k;
  int32_t index64;       // q_pos / kv_lens are int64
};

struct Lds {
  uint32_t hist[kRowsPerBlock][kBins];
  uint64_t cand[kRowsPerBlock][kCap];
};

// --------------------------------------------------------- wave primitives

__device__ __forceinline__ uint32_t shfl_xor_u32(uint32_t v, int m) {
  return (uint32_t)__shfl_xor((int)v, m, 64);
}
__device__ __forceinline__ uint64_t shfl_xor_u64(uint64_t v, int m) {
  return (uint64_t)shfl_xor_u32((uint32_t)v, m) | ((uint64_t)shfl_xor_u32((uint32_t)(v >> 32), m) << 32);
}
__device__ __forceinline__ uint32_t wave_sum_u32(uint32_t v) {
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) v += shfl_xor_u32(v, m);
  return v;
}
__device__ __forceinline__ float wave_max_f32(float v) {
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) v = __builtin_fmaxf(v, __uint_as_float(shfl_xor_u32(__float_as_uint(v), m)));
  return v;
}
__device__ __forceinline__ float wave_min_f32(float v) {
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) v = __builtin_fminf(v, __uint_as_float(shfl_xor_u32(__float_as_uint(v), m)));
  return v;
}
__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) {
    const uint64_t o = shfl_xor_u64(v, m);
    v = o > v ? o : v;
  }
  return v;
}
__device__ __forceinline__ uint64_t wave_min_u64(uint64_t v) {
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) {
    const uint64_t o = shfl_xor_u64(v, m);
    v = o < v ? o : v;
  }
  return v;
}
// Exclusive prefix sum over lanes 0..63.
__device__ __forceinline__ uint32_t wave_excl_scan(uint32_t v, int lane) {
  uint32_t x = v;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const uint32_t o = (uint32_t)__shfl_up((int)x, d, 64);
    if (lane >= d) x += o;
  }
  return x - v;
}

// ------------------------------------------------------------- row data

// Ordered key of an fp32 score: larger score -> larger key; -0 and +0 share
// one key.  (NaN is outside the contract.)
__device__ __forceinline__ uint32_t score_key(float v) {
  uint32_t u = __float_as_uint(v);
  u = v == 0.0f ? 0u : u;
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ uint64_t composite(uint32_t key, int id) {
  return ((uint64_t)key << 32) | (uint64_t)(0xffffffffu - (uint32_t)id);
}

// Element e of a lane: 16-byte vector e / VEC covers 64 * VEC consecutive
// blocks, the lane's VEC of them at lane * VEC.
template <bool BF16>
__device__ __forceinline__ int elem_id(int e, int lane) {
  constexpr int VEC = BF16 ? 8 : 4;
  return (e / VEC) * (64 * VEC) + lane * VEC + (e % VEC);
}

// ----------------------------------------------------------- bitonic sort

// Sorts the wave's 64 * EPS keys descending; lane l holds keys l * EPS ..
// l * EPS + EPS - 1 (strides below EPS are compared inside a lane, larger
// ones with the lane l ^ (stride / EPS)).
template <int EPS>
__device__ __forceinline__ void bitonic_sort_desc(uint64_t (&a)[EPS], int lane) {
  constexpr int N = 64 * EPS;
#pragma unroll
  for (int size = 2; size <= N; size <<= 1) {
#pragma unroll
    for (int d = size >> 1; d > 0; d >>= 1) {
      if (d < EPS) {
#pragma unroll
        for (int e = 0; e < EPS; ++e) {
          const int f = e ^ d;
          if (f > e) {
            const int i = lane * EPS + e;
            const bool desc = (i & size) == 0;
            const uint64_t x = a[e], y = a[f];
            const bool sw = desc ? (x < y) : (x > y);
            a[e] = sw ? y : x;
            a[f] = sw ? x : y;
          }
        }
      } else {
        const int m = d / EPS;
        const bool lower = (lane & m) == 0;
#pragma unroll
        for (int e = 0; e < EPS; ++e) {
          const int i = lane * EPS + e;
          const bool desc = (i & size) == 0;
          const uint64_t mine = a[e];
          const uint64_t other = shfl_xor_u64(mine, m);
          const bool take_max = lower == desc;
          a[e] = take_max ? (other > mine ? other : mine) : (other < mine ? other : mine);
        }
      }
    }
  }
}

template <int EPS>
__device__ __forceinline__ void sort_and_write(const uint64_t* cand, int nc, int lane,
                                               const DArgs& g, int64_t row, int b) {
  uint64_t a[EPS];
#pragma unroll
  for (int e = 0; e < EPS; ++e) {
    const int i = lane * EPS + e;
    a[e] = i < nc ? cand[i] : 0ull;     // 0 sorts below every selectable key
  }
  bitonic_sort_desc<EPS>(a, lane);
  const int K = g.top_k;
  const int take = nc < K ? nc : K;
#pragma unroll
  for (int e = 0; e < EPS; ++e) {
    const int t = lane * EPS + e;
    if (t < K) {
      int32_t blk = -1, page = -1;
      if (t < take) {
        blk = (int32_t)(0xffffffffu - (uint32_t)a[e]);
        page = g.page_table[(int64_t)b * g.NB + blk];
      }
      g.out_blocks[row * K + t] = blk;
      g.out_pages[row * K + t] = page;
    }
  }
  // Ranks past the sorted width (top_k > 64 * EPS >= the candidate count) are empty.
  for (int t = 64 * EPS + lane; t < K; t += 64) {
    g.out_blocks[row * K + t] = -1;
    g.out_pages[row * K + t] = -1;
  }
}

// ----------------------------------------------------------------- kernel

template <int EPL, bool BF16>
__global__ void __launch_bounds__(kThreads) dsa_topk_rows(const DArgs g) {
  constexpr int VEC = BF16 ? 8 : 4;
  static_assert(EPL % VEC == 0, "elements per lane");
  __shared__ Lds lds;
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t row = (int64_t)blockIdx.x * kRowsPerBlock + w;
  if (row >= g.rows) return;                 // whole wave leaves; no workgroup barrier below
  const int K = g.top_k;
  const int q = (int)(row % g.Q);
  const int b = (int)((row / g.Q) / g.H);
  const int64_t pos = g.index64 ? ((const int64_t*)g.q_pos)[(int64_t)b * g.Q + q]
                                : (int64_t)((const int32_t*)g.q_pos)[(int64_t)b * g.Q + q];
  const int64_t kv = g.index64 ? ((const int64_t*)g.kv_lens)[b]
                               : (int64_t)((const int32_t*)g.kv_lens)[b];
  int64_t vb = (kv + g.block_size - 1) / g.block_size;     // valid_blocks (kv >= 0)
  vb = vb < g.NB ? vb : g.NB;
  int64_t last = pos >= 0 ? pos / g.block_size : -1;
  last = last < vb - 1 ? last : vb - 1;
  const int nvalid = pos >= 0 && last >= 0 ? (int)(last + 1) : 0;

  // Scores of the valid prefix, rounded up to whole 16-byte vectors (inside
  // the row: NB is a multiple of VEC) so that no vector straddles the
  // descriptor's end; vectors past it read as zero.  Blocks past the prefix
  // are masked by id.
  constexpr uint32_t esz = BF16 ? 2u : 4u;
  const uint32_t nload = ((uint32_t)nvalid + VEC - 1) / VEC * VEC;
  const rsrc_t rs = make_rsrc((const uint8_t*)g.scores + row * (int64_t)g.NB * esz, nload * esz);
  float v[EPL];
#pragma unroll
  for (int i = 0; i < EPL / VEC; ++i) {
    const u32x4 d = __builtin_amdgcn_raw_buffer_load_b128(rs, (uint32_t)(i * 64 + lane) * 16u, 0, 0);
    if constexpr (BF16) {
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        v[i * 8 + 2 * c] = bf16_lo(d[c]);
        v[i * 8 + 2 * c + 1] = bf16_hi(d[c]);
      }
    } else {
#pragma unroll
      for (int c = 0; c < 4; ++c) v[i * 4 + c] = __uint_as_float(d[c]);
    }
  }
  auto selectable = [&](int e) {
    return elem_id<BF16>(e, lane) < nvalid && v[e] != -__builtin_inff();
  };

  uint32_t nsel = 0;
#pragma unroll
  for (int e = 0; e < EPL; ++e) nsel += selectable(e) ? 1u : 0u;
  nsel = wave_sum_u32(nsel);

  uint32_t* hist = lds.hist[w];
  uint64_t* cand = lds.cand[w];
  uint64_t lo = 0;                           // candidates: composite key >= lo

  if (nsel > (uint32_t)kCap) {
    // First split: 256 bins over the fp32 range of the selectable scores.
    float vmax = -__builtin_inff(), vmin = __builtin_inff();
#pragma unroll
    for (int e = 0; e < EPL; ++e)
      if (selectable(e)) {
        vmax = __builtin_fmaxf(vmax, v[e]);
        vmin = __builtin_fminf(vmin, v[e]);
      }
    vmax = wave_max_f32(vmax);
    vmin = wave_min_f32(vmin);
    const float scale = (float)kBins / (vmax - vmin);
    uint64_t hi = ~0ull;                     // search range [lo, hi] on the composite key
    uint32_t need = (uint32_t)K;             // still to find inside the range
    bool float_pass = vmax > vmin && __builtin_isfinite(scale) && __builtin_isfinite(vmin) &&
                      __builtin_isfinite(vmax);
    for (;;) {
      // Histogram of the in-range blocks (float bins on the first pass,
      // composite-key bins afterwards).
      uint64_t kmin = 0, width = 1;
      if (!float_pass) {
        uint64_t mn = ~0ull, mx = 0;
#pragma unroll
        for (int e = 0; e < EPL; ++e)
          if (selectable(e)) {
            const uint64_t c = composite(score_key(v[e]), elem_id<BF16>(e, lane));
            if (c >= lo && c <= hi) {
              mn = c < mn ? c : mn;
              mx = c > mx ? c : mx;
            }
          }
        kmin = wave_min_u64(mn);
        const uint64_t range = wave_max_u64(mx) - kmin;
        width = range / kBins + 1;           // bins 0 .. range / width (<= 255)
      }
#pragma unroll
      for (int i = 0; i < kBins / 64; ++i) hist[i * 64 + lane] = 0u;
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
#pragma unroll
      for (int e = 0; e < EPL; ++e)
        if (selectable(e)) {
          uint32_t bin;
          bool in = true;
          if (float_pass) {
            const float f = (v[e] - vmin) * scale;
            bin = f >= (float)(kBins - 1) ? (uint32_t)(kBins - 1) : (uint32_t)f;
          } else {
            const uint64_t c = composite(score_key(v[e]), elem_id<BF16>(e, lane));
            in = c >= lo && c <= hi;
            bin = in ? (uint32_t)((c - kmin) / width) : 0u;
          }
          if (in) __hip_atomic_fetch_add(&hist[bin], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WAVEFRONT);
        }
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      // Boundary bin: above(b) < need <= above(b) + hist[b], above(b) = blocks in higher bins.
      uint32_t hb[kBins / 64], lane_sum = 0;
#pragma unroll
      for (int i = 0; i < kBins / 64; ++i) {
        hb[i] = hist[lane * (kBins / 64) + i];
        lane_sum += hb[i];
      }
      uint32_t rev = 0;   // blocks in the bins of higher lanes (exclusive suffix sum)
      {
        uint32_t x = lane_sum;
#pragma unroll
        for (int dd = 1; dd < 64; dd <<= 1) {
          const uint32_t o = (uint32_t)__shfl_down((int)x, dd, 64);
          if (lane + dd < 64) x += o;
        }
        rev = x - lane_sum;
      }
      int bstar = -1;
      uint32_t above_star = 0, cnt_star = 0;
      {
        uint32_t above = rev;
#pragma unroll
        for (int i = kBins / 64 - 1; i >= 0; --i) {
          if (bstar < 0 && above < need && need <= above + hb[i]) {
            bstar = lane * (kBins / 64) + i;
            above_star = above;
            cnt_star = hb[i];
          }
          above += hb[i];
        }
      }
      const uint64_t ball = __ballot(bstar >= 0);
      const int src = __builtin_ctzll(ball);
      bstar = __shfl(bstar, src, 64);
      above_star = (uint32_t)__shfl((int)above_star, src, 64);
      cnt_star = (uint32_t)__shfl((int)cnt_star, src, 64);
      // New range: the composite keys of the boundary bin's blocks.
      uint64_t mn = ~0ull, mx = 0;
#pragma unroll
      for (int e = 0; e < EPL; ++e)
        if (selectable(e)) {
          const uint64_t c = composite(score_key(v[e]), elem_id<BF16>(e, lane));
          uint32_t bin;
          bool in = true;
          if (float_pass) {
            const float f = (v[e] - vmin) * scale;
            bin = f >= (float)(kBins - 1) ? (uint32_t)(kBins - 1) : (uint32_t)f;
          } else {
            in = c >= lo && c <= hi;
            bin = in ? (uint32_t)((c - kmin) / width) : 0u;
          }
          if (in && (int)bin == bstar) {
            mn = c < mn ? c : mn;
            mx = c > mx ? c : mx;
          }
        }
      const uint64_t new_lo = wave_min_u64(mn);
      const uint64_t new_hi = wave_max_u64(mx);
      // Blocks strictly above the new range are in the result: K - need
      // found before this pass plus above_star in this one.
      const uint32_t found = (uint32_t)K - need + above_star;
      lo = new_lo;
      hi = new_hi;
      if (found + cnt_star <= (uint32_t)kCap) break;
      need -= above_star;
      float_pass = false;
    }
  }

  // Compaction of the candidates (selectable, composite key >= lo).
  uint32_t mine = 0;
#pragma unroll
  for (int e = 0; e < EPL; ++e)
    if (selectable(e) && composite(score_key(v[e]), elem_id<BF16>(e, lane)) >= lo) ++mine;
  uint32_t off = wave_excl_scan(mine, lane);
  const uint32_t nc = wave_sum_u32(mine);
#pragma unroll
  for (int e = 0; e < EPL; ++e)
    if (selectable(e)) {
      const uint64_t c = composite(score_key(v[e]), elem_id<BF16>(e, lane));
      if (c >= lo) cand[off++] = c;
    }
  __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");

  const int n = (int)nc;
  if (n <= 64) sort_and_write<1>(cand, n, lane, g, row, b);
  else if (n <= 128) sort_and_write<2>(cand, n, lane, g, row, b);
  else if (n <= 256) sort_and_write<4>(cand, n, lane, g, row, b);
  else sort_and_write<8>(cand, n, lane, g, row, b);
}

using Kernel = void (*)(DArgs);

const void* kernel_for(int epl, bool bf16) {
  switch (epl) {
    case 8: return bf16 ? (const void*)&dsa_topk_rows<8, true> : (const void*)&dsa_topk_rows<8, false>;
    case 16: return bf16 ? (const void*)&dsa_topk_rows<16, true> : (const void*)&dsa_topk_rows<16, false>;
    case 32: return bf16 ? (const void*)&dsa_topk_rows<32, true> : (const void*)&dsa_topk_rows<32, false>;
    default: return bf16 ? (const void*)&dsa_topk_rows<64, true> : (const void*)&dsa_topk_rows<64, false>;
  }
}

bool aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }

}  // namespace
}  // namespace dsa
}  // namespace fagq

using namespace fagq;
using namespace fagq::dsa;

extern "C" {

FAGQ_API int fagq_dsa_topk_launch(const void* scores, int scores_dtype, const void* page_table,
                                  const void* q_pos, const void* kv_lens, int index_dtype,
                                  void* out_blocks, void* out_pages, int64_t B, int64_t H,
                                  int64_t Q, int64_t NB, int64_t block_size, int64_t top_k,
                                  void* stream) {
  if (!scores || !page_table || !q_pos || !kv_lens || !out_blocks || !out_pages)
    return FAGQ_E_NULL;
  if ((scores_dtype != FAGQ_DSA_F32 && scores_dtype != FAGQ_DSA_BF16) ||
      (index_dtype != FAGQ_DSA_I32 && index_dtype != FAGQ_DSA_I64))
    return FAGQ_E_FORMAT;
  if (B < 0 || H < 0 || Q < 0 || NB <= 0 || block_size < 1 || top_k < 1) return FAGQ_E_SHAPE;
  if (NB > FAGQ_DSA_MAX_NB || top_k > kMaxTopK || block_size > INT32_MAX) return FAGQ_E_TOO_LARGE;
  const int64_t rows = B * H * Q;
  const int64_t esz = scores_dtype == FAGQ_DSA_BF16 ? 2 : 4;
  if (rows > (int64_t)INT32_MAX * kRowsPerBlock || NB * esz > (int64_t)UINT32_MAX)
    return FAGQ_E_TOO_LARGE;
  if (!aligned(scores, 16) || (NB * esz) % 16 != 0 || !aligned(page_table, 4) ||
      !aligned(out_blocks, 4) || !aligned(out_pages, 4) ||
      !aligned(q_pos, index_dtype == FAGQ_DSA_I64 ? 8 : 4) ||
      !aligned(kv_lens, index_dtype == FAGQ_DSA_I64 ? 8 : 4))
    return FAGQ_E_ALIGN;
  if (rows == 0) return FAGQ_OK;
  const uintptr_t ob = reinterpret_cast<uintptr_t>(out_blocks), op = reinterpret_cast<uintptr_t>(out_pages);
  const uintptr_t on = (uintptr_t)(rows * top_k * 4);
  if (ob < op + on && op < ob + on) return FAGQ_E_ALIAS;
  const int dc = device_check();
  if (dc != FAGQ_OK) return dc;
  DArgs g;
  g.scores = scores;
  g.page_table = static_cast<const int32_t*>(page_table);
  g.q_pos = q_pos;
  g.kv_lens = kv_lens;
  g.out_blocks = static_cast<int32_t*>(out_blocks);
  g.out_pages = static_cast<int32_t*>(out_pages);
  g.rows = rows;
  g.H = (int32_t)H;
  g.Q = (int32_t)Q;
  g.NB = (int32_t)NB;
  g.block_size = (int32_t)block_size;
  g.top_k = (int32_t)top_k;
  g.index64 = index_dtype == FAGQ_DSA_I64;
  const bool bf16 = scores_dtype == FAGQ_DSA_BF16;
  const int64_t per_lane = (NB + 63) / 64;
  int epl = 8;
  while (epl < per_lane) epl <<= 1;
  void* args[] = {&g};
  const hipError_t e = hipLaunchKernel(kernel_for(epl, bf16),
                                       dim3((unsigned)((rows + kRowsPerBlock - 1) / kRowsPerBlock)),
                                       dim3(kThreads), args, 0, static_cast<hipStream_t>(stream));
  return e == hipSuccess ? FAGQ_OK : -(int)e;
}

}  // extern "C"
