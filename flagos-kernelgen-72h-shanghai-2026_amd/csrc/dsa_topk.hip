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
// Work mapping.  One workgroup per row, one wave per 1024 blocks of it (up
// to 4 waves); a lane holds 16 scores in VGPRs, loaded as 16-byte vectors
// through a buffer descriptor sized to the row's valid prefix, so blocks past
// it are never fetched.  Cross-lane steps use DPP and v_permlane16/32_swap
// (VALU, no LDS round trip); the waves of a row combine through a few LDS
// words and workgroup barriers, and every decision is computed identically
// by all of them.
//
// Selection is exact and never sorts the whole row:
//   * Every selectable block has a 32-bit ordered key of its score (larger
//     is better, -0 and +0 one key, 0 for blocks that are not selectable)
//     and a 64-bit composite key (key << 32) | (0xffffffff - id): the order
//     is score descending, then id ascending.
//   * If at most CAP (512) blocks are selectable they are all candidates.
//   * Otherwise a 256-bin histogram in LDS over the scores' fp32 range (the
//     bin is a monotone function of the score) locates the bin holding the
//     top_k-th block; with that bin and all higher ones at most CAP blocks,
//     those are the candidates.  Otherwise the bin becomes a search range
//     [lo, hi] on the composite key and is split again by 256-bin histograms
//     on the composite key, which always separate the range's smallest and
//     largest keys, so the loop ends.
//   * The candidates are compacted to LDS, bitonic-sorted in registers
//     across one wave (descending), and the first top_k are written with
//     their page-table entries.
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

constexpr int kEPL = 16;                    // scores per lane
constexpr int kChunk = 64 * kEPL;            // blocks per wave
constexpr int kMaxWaves = FAGQ_DSA_MAX_NB / kChunk;
constexpr int kBins = 256;
constexpr int kCap = 512;                    // candidates sorted at most
constexpr int kMaxTopK = FAGQ_DSA_MAX_TOP_K;
static_assert(kMaxWaves * kChunk == FAGQ_DSA_MAX_NB, "waves per row");

struct DArgs {
  const void* scores;
  const int32_t* page_table;
  const void* q_pos;
  const void* kv_lens;
  int32_t* out_blocks;
  int32_t* out_pages;
  int32_t H, Q, NB;
  int32_t block_size;
  int32_t top_k;
  int32_t index64;       // q_pos / kv_lens are int64
};

struct Lds {
  uint32_t hist[kBins];
  uint64_t cand[kCap];
  uint32_t slot[2][kMaxWaves][4];   // per-wave partials (two sets, alternating)
};

// --------------------------------------------------------- wave primitives

template <int CTRL>
__device__ __forceinline__ uint32_t dpp(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xf, 0xf, false);
}

// Value of lane (lane ^ m), m a power of two below 64.
__device__ __forceinline__ uint32_t xor_lane(uint32_t v, int m, int lane) {
  switch (m) {
    case 1: return dpp<0xB1>(v);                      // quad_perm [1,0,3,2]
    case 2: return dpp<0x4E>(v);                      // quad_perm [2,3,0,1]
    case 4: return (uint32_t)__builtin_amdgcn_ds_swizzle((int)v, 0x1F | (4 << 10));
    case 8: return (uint32_t)__builtin_amdgcn_ds_swizzle((int)v, 0x1F | (8 << 10));
    case 16: {
      const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
      return (lane & 16) ? r[0] : r[1];
    }
    default: {
      const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
      return (lane & 32) ? r[0] : r[1];
    }
  }
}
__device__ __forceinline__ uint64_t xor_lane64(uint64_t v, int m, int lane) {
  return (uint64_t)xor_lane((uint32_t)v, m, lane) |
         ((uint64_t)xor_lane((uint32_t)(v >> 32), m, lane) << 32);
}

// Reductions over the wave; every lane receives the result.  The first four
// steps reduce each 16-lane row (xor 1, xor 2, mirror in 8, mirror in 16),
// then the two permlane swaps join rows.
template <class Op>
__device__ __forceinline__ uint32_t wave_reduce(uint32_t v, Op op) {
  v = op(v, dpp<0xB1>(v));
  v = op(v, dpp<0x4E>(v));
  v = op(v, dpp<0x141>(v));
  v = op(v, dpp<0x140>(v));
  {
    const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
    v = op(r[0], r[1]);
  }
  {
    const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    v = op(r[0], r[1]);
  }
  return v;
}
template <class Op>
__device__ __forceinline__ uint64_t wave_reduce64(uint64_t v, Op op, int lane) {
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) v = op(v, xor_lane64(v, m, lane));
  return v;
}
struct Add { __device__ uint32_t operator()(uint32_t a, uint32_t b) const { return a + b; } };
struct Max { __device__ uint32_t operator()(uint32_t a, uint32_t b) const { return a > b ? a : b; } };
struct Min { __device__ uint32_t operator()(uint32_t a, uint32_t b) const { return a < b ? a : b; } };
struct Max64 { __device__ uint64_t operator()(uint64_t a, uint64_t b) const { return a > b ? a : b; } };
struct Min64 { __device__ uint64_t operator()(uint64_t a, uint64_t b) const { return a < b ? a : b; } };

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
// one key; every finite or infinite score except -inf maps above 0x007fffff.
__device__ __forceinline__ uint32_t score_key(float v) {
  uint32_t u = __float_as_uint(v);
  u = v == 0.0f ? 0u : u;
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float key_score(uint32_t k) {
  return __uint_as_float((k & 0x80000000u) ? (k ^ 0x80000000u) : ~k);
}

__device__ __forceinline__ uint64_t composite(uint32_t key, int id) {
  return ((uint64_t)key << 32) | (uint64_t)(0xffffffffu - (uint32_t)id);
}

// Block id of score e of a lane in wave w: 16-byte vector e / VEC covers
// 64 * VEC consecutive blocks, the lane's VEC of them at lane * VEC.
template <bool BF16>
__device__ __forceinline__ int elem_id(int e, int lane, int w) {
  constexpr int VEC = BF16 ? 8 : 4;
  return w * kChunk + (e / VEC) * (64 * VEC) + lane * VEC + (e % VEC);
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
            const bool desc = ((lane * EPS + e) & size) == 0;
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
          const bool desc = ((lane * EPS + e) & size) == 0;
          const uint64_t mine = a[e];
          const uint64_t other = xor_lane64(mine, m, lane);
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

// Workgroup-wide combine of one value per wave (all lanes of a wave hold
// it): lane 0 of each wave writes slot i of set `set`, a barrier, and every
// wave reads the nw values.
template <class Op>
__device__ __forceinline__ uint32_t group_combine(Lds& lds, int set, int i, uint32_t v, int w,
                                                  int nw, int lane, Op op, uint32_t ident) {
  if (lane == 0) lds.slot[set][w][i] = v;
  __syncthreads();
  uint32_t r = ident;
  for (int x = 0; x < nw; ++x) r = op(r, lds.slot[set][x][i]);
  return r;
}

template <bool BF16>
__global__ void __launch_bounds__(64 * kMaxWaves) dsa_topk_rows(const DArgs g) {
  constexpr int VEC = BF16 ? 8 : 4;
  __shared__ Lds lds;
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int nw = (int)(blockDim.x >> 6);
  const int64_t row = blockIdx.x;
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

  // Keys of the valid prefix.  The descriptor covers the prefix rounded up
  // to whole 16-byte vectors (inside the row: NB is a multiple of VEC), so no
  // vector straddles its end; vectors past it read as zero and blocks past
  // the prefix are masked by id.
  constexpr uint32_t esz = BF16 ? 2u : 4u;
  const uint32_t nload = ((uint32_t)nvalid + VEC - 1) / VEC * VEC;
  const rsrc_t rs = make_rsrc((const uint8_t*)g.scores + row * (int64_t)g.NB * esz, nload * esz);
  uint32_t key[kEPL];
#pragma unroll
  for (int i = 0; i < kEPL / VEC; ++i) {
    const u32x4 d = __builtin_amdgcn_raw_buffer_load_b128(
        rs, (uint32_t)(w * kChunk * esz) + (uint32_t)(i * 64 + lane) * 16u, 0, 0);
    float v[VEC];
    if constexpr (BF16) {
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        v[2 * c] = bf16_lo(d[c]);
        v[2 * c + 1] = bf16_hi(d[c]);
      }
    } else {
#pragma unroll
      for (int c = 0; c < 4; ++c) v[c] = __uint_as_float(d[c]);
    }
#pragma unroll
    for (int c = 0; c < VEC; ++c) {
      const int e = i * VEC + c;
      const bool sel = elem_id<BF16>(e, lane, w) < nvalid && v[c] != -__builtin_inff();
      key[e] = sel ? score_key(v[c]) : 0u;
    }
  }

  // Row totals: selectable count, largest key, smallest selectable key.
  uint32_t cnt = 0, kmax = 0, kmin = 0xffffffffu;
#pragma unroll
  for (int e = 0; e < kEPL; ++e) {
    cnt += key[e] != 0u;
    kmax = key[e] > kmax ? key[e] : kmax;
    kmin = key[e] != 0u && key[e] < kmin ? key[e] : kmin;
  }
  cnt = wave_reduce(cnt, Add());
  kmax = wave_reduce(kmax, Max());
  kmin = wave_reduce(kmin, Min());
  if (lane == 0) {
    lds.slot[0][w][0] = cnt;
    lds.slot[0][w][1] = kmax;
    lds.slot[0][w][2] = kmin;
  }
  __syncthreads();
  uint32_t nsel = 0;
  kmax = 0;
  kmin = 0xffffffffu;
  for (int x = 0; x < nw; ++x) {
    nsel += lds.slot[0][x][0];
    kmax = lds.slot[0][x][1] > kmax ? lds.slot[0][x][1] : kmax;
    kmin = lds.slot[0][x][2] < kmin ? lds.slot[0][x][2] : kmin;
  }

  // Candidate rule: mode 0 all selectable; 1 fp32 bin >= bstar; 2 composite >= lo.
  int mode = 0, bstar = 0;
  float vmin = 0.0f, scale = 0.0f;
  uint64_t lo = 0;
  int set = 1;
  if (nsel > (uint32_t)kCap) {
    const float fmax = key_score(kmax), fmin = key_score(kmin);
    vmin = fmin;
    scale = (float)kBins / (fmax - fmin);
    const bool float_ok = fmax > fmin && __builtin_isfinite(scale) && __builtin_isfinite(fmin) &&
                          __builtin_isfinite(fmax);
    uint64_t hi = ~0ull, kbase = 0, width = 1;
    uint32_t need = (uint32_t)K;
    bool float_pass = float_ok;
    for (;;) {
      auto fbin = [&](uint32_t k) {
        const float f = (key_score(k) - vmin) * scale;
        return f >= (float)(kBins - 1) ? (uint32_t)(kBins - 1) : (uint32_t)f;
      };
      if (!float_pass) {
        // Composite-key bins over the range [lo, hi].
        uint64_t mn = ~0ull, mx = 0;
#pragma unroll
        for (int e = 0; e < kEPL; ++e)
          if (key[e] != 0u) {
            const uint64_t c = composite(key[e], elem_id<BF16>(e, lane, w));
            if (c >= lo && c <= hi) {
              mn = c < mn ? c : mn;
              mx = c > mx ? c : mx;
            }
          }
        mn = wave_reduce64(mn, Min64(), lane);
        mx = wave_reduce64(mx, Max64(), lane);
        if (lane == 0) {
          lds.slot[set][w][0] = (uint32_t)mn;
          lds.slot[set][w][1] = (uint32_t)(mn >> 32);
          lds.slot[set][w][2] = (uint32_t)mx;
          lds.slot[set][w][3] = (uint32_t)(mx >> 32);
        }
        __syncthreads();
        mn = ~0ull;
        mx = 0;
        for (int x = 0; x < nw; ++x) {
          const uint64_t a = (uint64_t)lds.slot[set][x][0] | ((uint64_t)lds.slot[set][x][1] << 32);
          const uint64_t c = (uint64_t)lds.slot[set][x][2] | ((uint64_t)lds.slot[set][x][3] << 32);
          mn = a < mn ? a : mn;
          mx = c > mx ? c : mx;
        }
        set ^= 1;
        kbase = mn;
        width = (mx - mn) / kBins + 1;         // bins 0 .. (mx - mn) / width <= 255
      }
      auto bin_of = [&](int e, uint32_t& bin) {  // false: not in range
        if (key[e] == 0u) return false;
        if (float_pass) {
          bin = fbin(key[e]);
          return true;
        }
        const uint64_t c = composite(key[e], elem_id<BF16>(e, lane, w));
        if (c < lo || c > hi) return false;
        bin = (uint32_t)((c - kbase) / width);
        return true;
      };
      if (w == 0) {
#pragma unroll
        for (int i = 0; i < kBins / 64; ++i) lds.hist[i * 64 + lane] = 0u;
      }
      __syncthreads();
#pragma unroll
      for (int e = 0; e < kEPL; ++e) {
        uint32_t bin;
        if (bin_of(e, bin))
          __hip_atomic_fetch_add(&lds.hist[bin], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
      }
      __syncthreads();
      // Boundary bin: above(b) < need <= above(b) + hist[b], above(b) = blocks in higher bins.
      uint32_t hb[kBins / 64], lane_sum = 0;
#pragma unroll
      for (int i = 0; i < kBins / 64; ++i) {
        hb[i] = lds.hist[lane * (kBins / 64) + i];
        lane_sum += hb[i];
      }
      uint32_t incl = lane_sum;   // inclusive suffix sum over lanes >= lane
#pragma unroll
      for (int dd = 1; dd < 64; dd <<= 1) {
        const uint32_t o = (uint32_t)__shfl_down((int)incl, dd, 64);
        if (lane + dd < 64) incl += o;
      }
      int bs = -1;
      uint32_t above_s = 0, cnt_s = 0;
      {
        uint32_t above = incl - lane_sum;
#pragma unroll
        for (int i = kBins / 64 - 1; i >= 0; --i) {
          if (bs < 0 && above < need && need <= above + hb[i]) {
            bs = lane * (kBins / 64) + i;
            above_s = above;
            cnt_s = hb[i];
          }
          above += hb[i];
        }
      }
      const int src = __builtin_ctzll(__ballot(bs >= 0));
      bs = __shfl(bs, src, 64);
      above_s = (uint32_t)__shfl((int)above_s, src, 64);
      cnt_s = (uint32_t)__shfl((int)cnt_s, src, 64);
      const uint32_t found = (uint32_t)K - need + above_s;   // blocks above the boundary bin
      if (float_pass && found + cnt_s <= (uint32_t)kCap) {
        mode = 1;
        bstar = bs;
        break;
      }
      // The boundary bin's composite-key range.
      uint64_t mn = ~0ull, mx = 0;
#pragma unroll
      for (int e = 0; e < kEPL; ++e) {
        uint32_t bin;
        if (bin_of(e, bin) && (int)bin == bs) {
          const uint64_t c = composite(key[e], elem_id<BF16>(e, lane, w));
          mn = c < mn ? c : mn;
          mx = c > mx ? c : mx;
        }
      }
      mn = wave_reduce64(mn, Min64(), lane);
      mx = wave_reduce64(mx, Max64(), lane);
      if (lane == 0) {
        lds.slot[set][w][0] = (uint32_t)mn;
        lds.slot[set][w][1] = (uint32_t)(mn >> 32);
        lds.slot[set][w][2] = (uint32_t)mx;
        lds.slot[set][w][3] = (uint32_t)(mx >> 32);
      }
      __syncthreads();
      mn = ~0ull;
      mx = 0;
      for (int x = 0; x < nw; ++x) {
        const uint64_t a = (uint64_t)lds.slot[set][x][0] | ((uint64_t)lds.slot[set][x][1] << 32);
        const uint64_t c = (uint64_t)lds.slot[set][x][2] | ((uint64_t)lds.slot[set][x][3] << 32);
        mn = a < mn ? a : mn;
        mx = c > mx ? c : mx;
      }
      set ^= 1;
      lo = mn;
      hi = mx;
      if (found + cnt_s <= (uint32_t)kCap) {
        mode = 2;
        break;
      }
      need -= above_s;
      float_pass = false;
    }
  }

  // Compaction of the candidates into LDS.
  auto is_cand = [&](int e) {
    if (key[e] == 0u) return false;
    if (mode == 0) return true;
    if (mode == 1) {
      const float f = (key_score(key[e]) - vmin) * scale;
      const uint32_t bin = f >= (float)(kBins - 1) ? (uint32_t)(kBins - 1) : (uint32_t)f;
      return (int)bin >= bstar;
    }
    return composite(key[e], elem_id<BF16>(e, lane, w)) >= lo;
  };
  uint32_t mine = 0;
#pragma unroll
  for (int e = 0; e < kEPL; ++e) mine += is_cand(e);
  uint32_t off = wave_excl_scan(mine, lane);
  const uint32_t wtot = wave_reduce(mine, Add());
  if (lane == 0) lds.slot[set][w][0] = wtot;
  __syncthreads();
  uint32_t base = 0, nc = 0;
  for (int x = 0; x < nw; ++x) {
    const uint32_t t = lds.slot[set][x][0];
    base += x < w ? t : 0u;
    nc += t;
  }
  off += base;
#pragma unroll
  for (int e = 0; e < kEPL; ++e)
    if (is_cand(e)) lds.cand[off++] = composite(key[e], elem_id<BF16>(e, lane, w));
  __syncthreads();
  if (w != 0) return;

  const int n = (int)nc;
  if (n <= 64) sort_and_write<1>(lds.cand, n, lane, g, row, b);
  else if (n <= 128) sort_and_write<2>(lds.cand, n, lane, g, row, b);
  else if (n <= 256) sort_and_write<4>(lds.cand, n, lane, g, row, b);
  else sort_and_write<8>(lds.cand, n, lane, g, row, b);
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
  if (rows > (int64_t)INT32_MAX || NB * esz > (int64_t)UINT32_MAX)
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
  g.H = (int32_t)H;
  g.Q = (int32_t)Q;
  g.NB = (int32_t)NB;
  g.block_size = (int32_t)block_size;
  g.top_k = (int32_t)top_k;
  g.index64 = index_dtype == FAGQ_DSA_I64;
  const bool bf16 = scores_dtype == FAGQ_DSA_BF16;
  const int waves = (int)((NB + kChunk - 1) / kChunk);
  void* args[] = {&g};
  const void* k = bf16 ? (const void*)&dsa_topk_rows<true> : (const void*)&dsa_topk_rows<false>;
  const hipError_t e = hipLaunchKernel(k, dim3((unsigned)rows), dim3((unsigned)(64 * waves)), args,
                                       0, static_cast<hipStream_t>(stream));
  return e == hipSuccess ? FAGQ_OK : -(int)e;
}

}  // extern "C"
