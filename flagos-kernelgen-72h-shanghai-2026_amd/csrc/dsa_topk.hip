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
// Work mapping.  One workgroup per row, one wave per 1024-block chunk of it
// (up to 16 waves); a lane holds 16 scores in VGPRs, loaded through a buffer
// descriptor sized to the row's valid prefix, so blocks past it are never
// fetched, and waves wholly past the prefix exit at once (a workgroup barrier
// waits only for the waves still running); for top_k > 256 they stay idle
// until the rank phase and share its candidates.  Rows whose base is 16-byte
// aligned (scores pointer aligned and NB * element size a multiple of 16) are
// read as 16-byte vectors, other rows one score per load.  A row of more than
// 16 chunks (NB > 16384) is walked in chunks of 16 x 1024 blocks, each wave
// taking every 16th chunk and reading the scores again in each pass (the row
// is L2-resident after the first).  Cross-lane steps use DPP and
// v_permlane32_swap; the waves of a row combine through LDS and five
// workgroup barriers.
//
// Selection is exact and never runs a sorting network:
//   1. The fp32 range [vmin, vmax] of the selectable scores (non-selectable
//      blocks hold -inf) defines 255 bins, bin(v) = round(clamp(v s + c, 0,
//      255)) with s = 255 / (vmax - vmin), c = 1.5 - vmin s: a monotone
//      function of the score, 0 only for -inf (one fma and one
//      v_cvt_pk_u8_f32, which also packs four bins per word).
//   2. An LDS histogram of the bins; its suffix sums above(b) (blocks in
//      higher bins) give the boundary bin b* holding the top_k-th block.
//      The candidates are the blocks of bins >= b*: found = above(b*) of them
//      are certainly selected, and all of them fit in CAP (512 for top_k
//      <= 256, 2048 for larger top_k up to 1024; CAP >= top_k always).
//   3. Counting sort: a candidate is stored at its bin's cursor, which starts
//      at above(bin), so each bin owns one segment of the candidate array,
//      bins in descending order.  A candidate's rank is above(bin) plus the
//      number of candidates in its own segment that precede it (64-bit composite key:
//      (ordered score bits << 32) | (0xffffffff - id)); for Gaussian-like
//      scores a segment holds a few blocks.  Ranks below top_k are written
//      with their page-table entries.
//   If the boundary bin leaves more than CAP candidates (ties, outliers that
//   stretch the range), a refinement finds a threshold on the composite key
//   by 8-bit radix passes over the key range that remains, and the rank is
//   then counted over all candidates.  Composite keys are distinct, so the
//   passes end with at most top_k <= CAP keys at or above the threshold.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "fagq.h"
#include "fagq_dispatch.hpp"
#include "fagq_dsa.h"

namespace fagq {
namespace dsa {
namespace {

constexpr int kEPL = 16;                    // scores per lane
constexpr int kChunk = 64 * kEPL;            // blocks per wave chunk
constexpr int kMaxWaves = 16;                // waves per row (NB <= 16384 in one chunk each)
constexpr int kBins = 256;
// Candidates held at most: kCapSmall for top_k <= kSmallTopK, else kCapLarge.
constexpr uint32_t kCapSmall = 512;
constexpr uint32_t kCapLarge = 2048;
constexpr int kSmallTopK = 256;
constexpr int kMaxTopK = FAGQ_DSA_MAX_TOP_K;
static_assert(kMaxTopK <= (int)kCapLarge && kSmallTopK <= (int)kCapSmall, "top_k fits CAP");
constexpr int64_t kMaxGridYZ = 65535;        // H and B are grid dimensions y and z

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
  // n / block_size for n < 2^32 (Granlund-Montgomery, unsigned):
  // t = mulhi(bs_mul, n), n / block_size = (t + ((n - t) >> bs_sh1)) >> bs_sh2.
  uint32_t bs_mul, bs_sh1, bs_sh2;
};

__device__ __forceinline__ uint32_t div_bs(const DArgs& g, uint32_t n) {
  const uint32_t t = __umulhi(g.bs_mul, n);
  return (t + ((n - t) >> g.bs_sh1)) >> g.bs_sh2;
}

template <uint32_t CAP>
struct Lds {
  uint32_t hist[kBins + 64];        // bin counts, then one discard word per lane
  uint32_t above[kBins];            // 8 x candidates in higher bins: cand byte offsets, then
                                    // the scatter's per-bin cursors
  uint64_t cand[CAP + 4];           // 4 spare entries: the rank loop reads in fours
  uint32_t kslot[kMaxWaves][2];     // per-wave max / min (ord_key)
  uint32_t uslot[2][kMaxWaves][4];  // per-wave partials of the refinement
  uint32_t ncur;                    // refinement scatter cursor
  uint32_t bnd[2];                  // candidate count and boundary bin, from wave 0
};
constexpr int kZeroWords = kBins + 64;   // hist, cleared per row
static_assert(kZeroWords % 4 == 0, "cleared with 16-byte stores");

// --------------------------------------------------------- wave primitives

template <int CTRL, int ROW_MASK = 0xf>
__device__ __forceinline__ uint32_t dpp(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, ROW_MASK, 0xf, true);
}

// All-lane reduction: xor 1, xor 2 (quad permutes), mirror in 8, mirror in
// 16 reduce each 16-lane row; v_permlane16_swap and v_permlane32_swap join
// the rows.
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
struct UMax {
  __device__ uint32_t operator()(uint32_t a, uint32_t b) const { return a > b ? a : b; }
};
struct UMin {
  __device__ uint32_t operator()(uint32_t a, uint32_t b) const { return a < b ? a : b; }
};

// Order-preserving uint32 image of a non-NaN fp32 value (a < b implies
// ord_key(a) < ord_key(b); -0 sorts just below +0) and its inverse.  Wave and
// workgroup min / max run on these keys: one integer op per step, where fp32
// fmaxf / fminf would also quiet their operands.
__device__ __forceinline__ uint32_t ord_key(float v) {
  const uint32_t u = __float_as_uint(v);
  return u ^ ((uint32_t)((int32_t)u >> 31) | 0x80000000u);
}
__device__ __forceinline__ float ord_val(uint32_t k) {
  return __uint_as_float(k ^ (~(uint32_t)((int32_t)k >> 31) | 0x80000000u));
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
template <bool MAX>
__device__ __forceinline__ uint64_t wave_reduce64(uint64_t v, int lane) {
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) {
    const uint64_t o = (uint64_t)xor_lane((uint32_t)v, m, lane) |
                       ((uint64_t)xor_lane((uint32_t)(v >> 32), m, lane) << 32);
    v = MAX ? (o > v ? o : v) : (o < v ? o : v);
  }
  return v;
}

// Inclusive prefix sum over lanes 0..63: shifts 1, 2, 4, 8 inside each
// 16-lane row, then row_bcast:15 (rows 1 and 3 add the last lane of rows 0
// and 2) and row_bcast:31 (rows 2 and 3 add lane 31).
__device__ __forceinline__ uint32_t wave_incl_scan(uint32_t x) {
  x += dpp<0x111>(x);
  x += dpp<0x112>(x);
  x += dpp<0x114>(x);
  x += dpp<0x118>(x);
  x += dpp<0x142, 0xa>(x);
  x += dpp<0x143, 0xc>(x);
  return x;
}

// ------------------------------------------------------------- row data

// Ordered key of an fp32 score: larger score -> larger key; -0 and +0 share
// one key; every score except -inf maps above 0x007fffff.
__device__ __forceinline__ uint32_t score_key(float v) {
  uint32_t u = __float_as_uint(v);
  u = v == 0.0f ? 0u : u;
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float key_score(uint32_t k) {
  return __uint_as_float((k & 0x80000000u) ? (k ^ 0x80000000u) : ~k);
}
__device__ __forceinline__ uint64_t composite(float v, uint32_t id) {
  return ((uint64_t)score_key(v) << 32) | (uint64_t)(0xffffffffu - id);
}

// Histogram bin of a score under the linear map of [vmin, vmax]: s = 255 /
// (vmax - vmin), finite and positive, and c = fma(-vmin, s, 1.5) with
// |vmin s| < 2^21.  x = fma(v, s, c) is then within 0.125 of
// (v - vmin) s + 1.5, and v_cvt_pk_u8_f32 rounds it to the nearest integer
// clamped to [0, 255] (-inf -> 0), written into byte `byte` of `word`.  The
// bin is non-decreasing in v; a selectable score (v >= vmin) gets a bin in
// [1, 255] (x >= 1.375) and -inf gets bin 0.
__device__ __forceinline__ uint32_t fbin_pack(float v, float s, float c, uint32_t byte,
                                              uint32_t word) {
  return __builtin_amdgcn_cvt_pk_u8_f32(fmaf(v, s, c), byte, word);
}
__device__ __forceinline__ uint32_t fbin(float v, float s, float c) {
  return fbin_pack(v, s, c, 0u, 0u);
}
constexpr float kMaxBinOffset = 2097152.0f;   // 2^21: bound on |vmin s| for the map above

template <bool B>
struct BoolC {
  static constexpr bool value = B;
};

// Block id of score e of a lane in wave w: 16-byte vector e / VEC covers
// 64 * VEC consecutive blocks, the lane's VEC of them at lane * VEC.
template <bool BF16>
__device__ __forceinline__ int elem_off(int e) {
  constexpr int VEC = BF16 ? 8 : 4;
  return (e / VEC) * (64 * VEC) + (e % VEC);
}

// Boundary of a histogram in hist[0..255]: the bin b with
// above(b) < need <= above(b) + hist[b], above(b) = count in bins > b.
// Every lane receives bin, above(bin), hist[bin] and the histogram total.
// STORE marks the fp32-bin histogram: its bin 0 (non-selectable blocks) is
// left out, and, where `store`, 8 above(b) (the byte offset of bin b's
// segment of lds.cand) is written to lds.above.
struct Boundary {
  uint32_t bin, above, cnt, total;
};
template <bool STORE, class L>
__device__ __forceinline__ Boundary find_boundary(L& lds, uint32_t k, int lane,
                                                  bool store = false) {
  u32x4 h = reinterpret_cast<const u32x4*>(lds.hist)[lane];   // bins 4 lane .. 4 lane + 3
  if (STORE && lane == 0) h[0] = 0u;     // fp32 bins: bin 0 counts non-selectable blocks
  const uint32_t sum = h[0] + h[1] + h[2] + h[3];
  const uint32_t incl = wave_incl_scan(sum);
  Boundary r;
  r.total = (uint32_t)__builtin_amdgcn_readlane((int)incl, 63);
  const uint32_t need = k < r.total ? k : r.total;
  u32x4 a;
  a[3] = r.total - incl;
  a[2] = a[3] + h[3];
  a[1] = a[2] + h[2];
  a[0] = a[1] + h[1];
  if constexpr (STORE)
    if (store)
      reinterpret_cast<u32x4*>(lds.above)[lane] = u32x4{8u * a[0], 8u * a[1], 8u * a[2], 8u * a[3]};
  uint32_t bin = 0, ab = 0, cb = 0;
  bool hit = false;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const bool c = a[i] < need && need <= a[i] + h[i];
    bin = c ? (uint32_t)(4 * lane + i) : bin;
    ab = c ? a[i] : ab;
    cb = c ? h[i] : cb;
    hit = hit || c;
  }
  const uint64_t m = __ballot(hit);
  const int src = m ? __builtin_ctzll(m) : 0;
  r.bin = (uint32_t)__builtin_amdgcn_readlane((int)bin, src);
  r.above = m ? (uint32_t)__builtin_amdgcn_readlane((int)ab, src) : 0u;
  r.cnt = m ? (uint32_t)__builtin_amdgcn_readlane((int)cb, src) : 0u;
  return r;
}

// Score c of a 16-byte vector (c < 8 for bf16, c < 4 for fp32).
template <bool BF16>
__device__ __forceinline__ float vec_elem(const u32x4& d, int c) {
  if constexpr (BF16) return c % 2 ? bf16_hi(d[c / 2]) : bf16_lo(d[c / 2]);
  else return __uint_as_float(d[c]);
}

// ----------------------------------------------------------------- kernel

// One 16-byte vector of scores at byte offset `off` of the row (VEC scores:
// blocks off / esz .. + VEC - 1).  VECLD: one 16-byte load (rows 16-byte
// aligned, the descriptor covering the prefix rounded up to whole vectors
// inside the row); else one load per score through a descriptor sized to the
// prefix exactly, so scores past it read as 0 (and are then masked by the
// caller).
template <bool BF16, bool VECLD>
__device__ __forceinline__ u32x4 load_vec(const rsrc_t& rs, uint32_t off) {
  if constexpr (VECLD) {
    return __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, 0);
  } else {
    u32x4 v;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      if constexpr (BF16) {
        const uint32_t lo = __builtin_amdgcn_raw_buffer_load_b16(rs, off + 4u * c, 0, 0);
        const uint32_t hi = __builtin_amdgcn_raw_buffer_load_b16(rs, off + 4u * c + 2u, 0, 0);
        v[c] = lo | (hi << 16);
      } else {
        v[c] = __builtin_amdgcn_raw_buffer_load_b32(rs, off + 4u * c, 0, 0);
      }
    }
    return v;
  }
}

// The 16 scores of a lane in the chunk starting at block wbase: vector i
// holds blocks wbase + i * 64 * VEC + lane * VEC + c, c < VEC.
template <bool BF16, bool VECLD>
__device__ __forceinline__ void load_chunk(const rsrc_t& rs, int wbase, int lane,
                                           u32x4 (&raw)[kEPL / (BF16 ? 8 : 4)]) {
  constexpr int VEC = BF16 ? 8 : 4;
  constexpr uint32_t esz = BF16 ? 2u : 4u;
#pragma unroll
  for (int i = 0; i < kEPL / VEC; ++i)
    raw[i] = load_vec<BF16, VECLD>(rs, (uint32_t)(wbase * esz) + (uint32_t)(i * 64 + lane) * 16u);
}

// Scores of a loaded chunk: blocks at or past the prefix (rel = nvalid -
// wbase blocks remain) become -inf.  Updates the lane's maximum and the
// minimum over its selectable (not -inf) scores.
template <bool BF16, bool FULL>
__device__ __forceinline__ void chunk_scores(const u32x4 (&raw)[kEPL / (BF16 ? 8 : 4)], int lbase,
                                             int rel, float (&sv)[kEPL], float& vmin,
                                             float& vmax) {
  constexpr int VEC = BF16 ? 8 : 4;
  const float ninf = -__builtin_inff();
  float lmin = __builtin_inff();
#pragma unroll
  for (int i = 0; i < kEPL / VEC; ++i) {
#pragma unroll
    for (int c = 0; c < VEC; ++c) {
      const int e = i * VEC + c;
      const float v = vec_elem<BF16>(raw[i], c);
      sv[e] = FULL || lbase < rel - elem_off<BF16>(e) ? v : ninf;
      vmax = fmaxf(vmax, sv[e]);
      // A full chunk takes the plain minimum and redoes it below in the rare
      // case that an explicit -inf score made it -inf.
      if constexpr (FULL) lmin = fminf(lmin, sv[e]);
      else lmin = fminf(lmin, sv[e] != ninf ? sv[e] : __builtin_inff());
    }
  }
  if (FULL && lmin == ninf) {
    lmin = __builtin_inff();
#pragma unroll
    for (int e = 0; e < kEPL; ++e) lmin = fminf(lmin, sv[e] != ninf ? sv[e] : __builtin_inff());
  }
  vmin = fminf(vmin, lmin);
}

// KIND: kSmallRows (at most 4 chunks, 256-thread workgroups) or kRows (at
// most 16) keep one chunk per wave in VGPRs from the first pass to the last;
// kLongRows (more than 16 chunks): every wave walks chunks w, w + nwv, ... in
// each pass, reading its scores again.
enum RowKind { kSmallRows = 0, kRows = 1, kLongRows = 2 };
constexpr int kSmallWaves = 4;

template <bool BF16, bool VECLD, int KIND, uint32_t CAP>
__global__ void __launch_bounds__(KIND == kSmallRows ? 64 * kSmallWaves : 64 * kMaxWaves)
dsa_topk_rows(const DArgs g) {
  constexpr bool MULTI = KIND == kLongRows;
  constexpr int VEC = BF16 ? 8 : 4;
  __shared__ Lds<CAP> lds;
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  // Grid (Q, H, B): row = (b * H + h) * Q + q.
  const int q = (int)blockIdx.x;
  const int b = (int)blockIdx.z;
  const int64_t row = ((int64_t)b * g.H + (int64_t)blockIdx.y) * g.Q + q;
  const int K = g.top_k;
  const int64_t pos = g.index64 ? ((const int64_t*)g.q_pos)[(int64_t)b * g.Q + q]
                                : (int64_t)((const int32_t*)g.q_pos)[(int64_t)b * g.Q + q];
  const int64_t kv = g.index64 ? ((const int64_t*)g.kv_lens)[b]
                               : (int64_t)((const int32_t*)g.kv_lens)[b];
  // nvalid = last_block + 1, last_block = min(pos / bs, valid_blocks - 1),
  // valid_blocks = min(ceil(kv / bs), NB); 0 when pos < 0 or kv == 0.
  int nvalid = 0;
  if (pos >= 0 && kv > 0) {
    int64_t vb, lastp;
    if (pos <= INT32_MAX && kv <= INT32_MAX) {      // 32-bit operands (bs < 2^31)
      vb = div_bs(g, (uint32_t)kv + (uint32_t)g.block_size - 1u);
      lastp = div_bs(g, (uint32_t)pos);
    } else {
      vb = (kv - 1) / g.block_size + 1;
      lastp = pos / g.block_size;
    }
    vb = vb < g.NB ? vb : g.NB;
    nvalid = (int)(lastp < vb - 1 ? lastp : vb - 1) + 1;
  }
  const int nchunk = nvalid > kChunk ? (nvalid + kChunk - 1) / kChunk : 1;
  const int nwv = nchunk < (int)(blockDim.x >> 6) ? nchunk : (int)(blockDim.x >> 6);  // waves with work
  // top_k > kSmallTopK: the waves past the prefix stay for the rank phase,
  // where the candidates (up to CAP) outnumber the live waves' lanes; they
  // skip the score, histogram and scatter work (their chunks lie wholly past
  // the prefix) and take part in every barrier.  For smaller top_k they
  // leave at once.
  constexpr bool KEEP = CAP != kCapSmall && !MULTI;
  const bool live = w < nwv;
  if (!KEEP && !live) return;

  if (w == 0) {
    u32x4* z = reinterpret_cast<u32x4*>(lds.hist);
    for (int i = lane; i < kZeroWords / 4; i += 64) z[i] = u32x4{0u, 0u, 0u, 0u};
    if (lane == 0) lds.ncur = 0u;
  }

  // Scores of the valid prefix; non-selectable blocks hold -inf.  With vector
  // loads the descriptor covers the prefix rounded up to whole 16-byte vectors
  // (inside the row: NB is a multiple of VEC), so no vector straddles its end;
  // with per-score loads it covers the prefix exactly.  A chunk whose blocks
  // all lie in the prefix skips the per-block id test.
  constexpr uint32_t esz = BF16 ? 2u : 4u;
  const uint32_t nload = VECLD ? ((uint32_t)nvalid + VEC - 1) / VEC * VEC : (uint32_t)nvalid;
  const rsrc_t rs = make_rsrc((const uint8_t*)g.scores + row * (int64_t)g.NB * esz, nload * esz);
  const int lbase = lane * VEC;                  // lane's first block inside a vector span
  const float ninf = -__builtin_inff();
  float sv[kEPL];
  float vmax = ninf, vmin = __builtin_inff();
  // Runs f(wbase) for each chunk of this wave with sv holding its scores.
  auto each_chunk = [&](auto&& f) {
#pragma unroll 1
    for (int ci = w; ci < nchunk; ci += nwv) {
      const int wbase = ci * kChunk;
      u32x4 raw[kEPL / VEC];
      load_chunk<BF16, VECLD>(rs, wbase, lane, raw);
      float lo = __builtin_inff(), hi = ninf;
      if (wbase + kChunk <= nvalid) chunk_scores<BF16, true>(raw, lbase, nvalid - wbase, sv, lo, hi);
      else chunk_scores<BF16, false>(raw, lbase, nvalid - wbase, sv, lo, hi);
      f(wbase, wbase + kChunk <= nvalid, lo, hi);
    }
  };
  const int wbase0 = w * kChunk;               // the wave's chunk when !MULTI
  const bool full0 = wbase0 + kChunk <= nvalid;
  if constexpr (MULTI) {
    each_chunk([&](int, bool, float lo, float hi) {
      vmin = fminf(vmin, lo);
      vmax = fmaxf(vmax, hi);
    });
  } else if (live) {
    // Every load is issued before the full / partial split.
    u32x4 raw[kEPL / VEC];
    load_chunk<BF16, VECLD>(rs, wbase0, lane, raw);
    if (full0) chunk_scores<BF16, true>(raw, lbase, nvalid - wbase0, sv, vmin, vmax);
    else chunk_scores<BF16, false>(raw, lbase, nvalid - wbase0, sv, vmin, vmax);
  }
  uint32_t kmax = wave_reduce(ord_key(vmax), UMax());
  uint32_t kmin = wave_reduce(ord_key(vmin), UMin());
  if (lane == 0) {
    lds.kslot[w][0] = kmax;
    lds.kslot[w][1] = kmin;
  }
  __syncthreads();
  for (int x = 0; x < nwv; ++x) {
    kmax = kmax > lds.kslot[x][0] ? kmax : lds.kslot[x][0];
    kmin = kmin < lds.kslot[x][1] ? kmin : lds.kslot[x][1];
  }
  vmax = ord_val(kmax);
  vmin = ord_val(kmin);

  // Bin map (see fbin); a degenerate or non-finite range, or one too narrow
  // for its offset (|vmin s| >= 2^21), puts every selectable score in bin 1.
  // s needs no correct rounding: the histogram and the ranks use the same s
  // and c, and x(vmax) stays within rounding of 256.5, which clamps to 255.
  const float s = (float)(kBins - 1) * __builtin_amdgcn_rcpf(vmax - vmin);
  const float c = fmaf(-vmin, s, 1.5f);
  const bool degen = !(vmax > vmin) || !(s > 0.0f) || !__builtin_isfinite(s) ||
                     !(fabsf(vmin * s) < kMaxBinOffset);
  // Bins of the lane's scores, four 8-bit bins per word (0: not selectable).
  // Non-selectable blocks count in bin 0 (ignored) in a full chunk, where
  // they are rare, else in the lane's own discard word.
  uint32_t pbin[kEPL / 4];
  auto bins = [&](auto binf) {
#pragma unroll
    for (int e = 0; e < kEPL; ++e)
      pbin[e / 4] = binf(sv[e], (uint32_t)(e % 4), e % 4 ? pbin[e / 4] : 0u);
  };
  auto bin_lin = [=](float v, uint32_t byte, uint32_t word) {
    return fbin_pack(v, s, c, byte, word);
  };
  auto bin_one = [=](float v, uint32_t byte, uint32_t word) {
    return word | ((v != ninf ? 1u : 0u) << (8 * byte));
  };
  auto make_bins = [&]() {
    if (!degen) bins(bin_lin);
    else bins(bin_one);
  };
  auto hist = [&](auto full_c) {
#pragma unroll
    for (int e = 0; e < kEPL; ++e) {
      const uint32_t bn = (pbin[e / 4] >> (8 * (e % 4))) & 0xffu;
      const uint32_t at = decltype(full_c)::value || bn ? bn : (uint32_t)(kBins + lane);
      __hip_atomic_fetch_add(&lds.hist[at], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    }
  };
  auto hist_rt = [&](bool full) {
    if (full) hist(BoolC<true>());
    else hist(BoolC<false>());
  };
  if constexpr (MULTI) {
    each_chunk([&](int, bool full, float, float) {
      make_bins();
      hist(BoolC<false>());
      (void)full;
    });
  } else if (live) {
    make_bins();
    hist_rt(full0);
  }
  __syncthreads();

  // Wave 0 finds the boundary, stores above(b) and hands the candidate count
  // and the boundary bin to the other waves.
  uint32_t nc = 0, bstar = 1;
  if (w == 0) {
    const Boundary bd = find_boundary<true>(lds, (uint32_t)K, lane, true);
    nc = bd.total ? bd.above + bd.cnt : 0u;
    bstar = bd.bin > 1u ? bd.bin : 1u;
    if (lane == 0) {
      lds.bnd[0] = nc;
      lds.bnd[1] = bstar;
    }
  }
  __syncthreads();
  if (w != 0) {
    nc = (uint32_t)__builtin_amdgcn_readfirstlane((int)lds.bnd[0]);
    bstar = (uint32_t)__builtin_amdgcn_readfirstlane((int)lds.bnd[1]);
  }
  const bool refine = nc > CAP;

  if (!refine) {
    // Counting-sort scatter of the blocks in bins >= b* (b* >= 1, so bin 0,
    // the non-selectable blocks, never qualifies); p < nc <= CAP.  The entry
    // holds the raw score bits and 0xffffffff - id; the scores become ordered
    // keys in one pass over the candidates below.
    auto scatter = [&](int wbase) {
      const uint32_t nid = 0xffffffffu - (uint32_t)(wbase + lbase);
#pragma unroll
      for (int e = 0; e < kEPL; ++e) {
        const uint32_t bn = (pbin[e / 4] >> (8 * (e % 4))) & 0xffu;
        if (bn >= bstar) {
          // The cursor returns the entry's byte offset; a bin's slots end at
          // 8 (above(b*) + hist[b*]) = 8 nc <= 8 CAP, so no mask is needed.
          const uint32_t off = __hip_atomic_fetch_add(&lds.above[bn], 8u, __ATOMIC_RELAXED,
                                                      __HIP_MEMORY_SCOPE_WORKGROUP);
          const uint32_t lo = nid - (uint32_t)elem_off<BF16>(e);
          *reinterpret_cast<uint64_t*>(reinterpret_cast<uint8_t*>(lds.cand) + off) =
              ((uint64_t)__float_as_uint(sv[e]) << 32) | (uint64_t)lo;
        }
      }
    };
    if constexpr (MULTI) {
      each_chunk([&](int wbase, bool, float, float) {
        make_bins();
        scatter(wbase);
      });
    } else {
      if (live) scatter(wbase0);
    }
  } else {
    // Radix refinement on the composite key over [lo, hi]: found blocks lie
    // above hi, need more inside the range.  The scores are read again from
    // memory on each pass (this path is rare), so none stay live in VGPRs.
    auto keys = [&](auto&& f) {
#pragma unroll 1
      for (int ci = w; ci < nchunk; ci += nwv) {
        const int wbase = ci * kChunk;
#pragma unroll 1
        for (int i = 0; i < kEPL / VEC; ++i) {
          const u32x4 d = load_vec<BF16, VECLD>(
              rs, (uint32_t)(wbase * esz) + (uint32_t)(i * 64 + lane) * 16u);
#pragma unroll
          for (int cc = 0; cc < VEC; ++cc) {
            const float v = vec_elem<BF16>(d, cc);
            const int off = i * (64 * VEC) + cc;
            if (lbase < nvalid - wbase - off && v != ninf)
              f(composite(v, (uint32_t)(wbase + lbase + off)));
          }
        }
      }
    };
    auto uni = [](uint64_t x) {
      return (uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)x) |
             ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(x >> 32)) << 32);
    };
    uint64_t lo = 1, hi = ~0ull, thr = 1;
    uint32_t need = (uint32_t)K, found = 0;
    int set = 0;
    for (;;) {
      uint64_t mn = ~0ull, mx = 0;
      keys([&](uint64_t c) {
        if (c >= lo && c <= hi) {
          mn = c < mn ? c : mn;
          mx = c > mx ? c : mx;
        }
      });
      mn = wave_reduce64<false>(mn, lane);
      mx = wave_reduce64<true>(mx, lane);
      if (lane == 0) {
        lds.uslot[set][w][0] = (uint32_t)mn;
        lds.uslot[set][w][1] = (uint32_t)(mn >> 32);
        lds.uslot[set][w][2] = (uint32_t)mx;
        lds.uslot[set][w][3] = (uint32_t)(mx >> 32);
      }
      __syncthreads();
      mn = ~0ull;
      mx = 0;
      for (int x = 0; x < nwv; ++x) {
        const uint64_t a = (uint64_t)lds.uslot[set][x][0] | ((uint64_t)lds.uslot[set][x][1] << 32);
        const uint64_t c = (uint64_t)lds.uslot[set][x][2] | ((uint64_t)lds.uslot[set][x][3] << 32);
        mn = a < mn ? a : mn;
        mx = c > mx ? c : mx;
      }
      mn = uni(mn);
      mx = uni(mx);
      set ^= 1;
      // 8-bit digit at the highest bit where mn and mx differ: they fall in
      // different bins, so every pass shrinks the range.
      const int hb = mn == mx ? 0 : 63 - __builtin_clzll(mn ^ mx);
      const int shift = hb > 7 ? hb - 7 : 0;
      const uint64_t base = mn >> shift;
      if (w == 0) reinterpret_cast<u32x4*>(lds.hist)[lane] = u32x4{0u, 0u, 0u, 0u};
      __syncthreads();
      keys([&](uint64_t c) {
        if (c >= lo && c <= hi)
          __hip_atomic_fetch_add(&lds.hist[(uint32_t)((c >> shift) - base)], 1u, __ATOMIC_RELAXED,
                                 __HIP_MEMORY_SCOPE_WORKGROUP);
      });
      __syncthreads();
      const Boundary r = find_boundary<false>(lds, need, lane);
      thr = (base + r.bin) << shift;
      if (found + r.above + r.cnt <= CAP) {
        nc = found + r.above + r.cnt;
        break;
      }
      const uint64_t top = base + r.bin + 1;
      if (shift + (64 - __builtin_clzll(top)) <= 64) {
        const uint64_t h2 = (top << shift) - 1;
        hi = h2 < hi ? h2 : hi;
      }
      lo = thr;
      need -= r.above;
      found += r.above;
    }
    keys([&](uint64_t c) {
      if (c >= thr) {
        const uint32_t p =
            __hip_atomic_fetch_add(&lds.ncur, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        if (p < CAP) lds.cand[p] = c;
      }
    });
  }
  __syncthreads();

  const int stride = KEEP ? (int)blockDim.x : 64 * nwv;
  const int t = w * 64 + lane;
  if (!refine) {
    for (uint32_t i = (uint32_t)t; i < nc; i += (uint32_t)stride) {
      const uint64_t c = lds.cand[i];
      lds.cand[i] = ((uint64_t)score_key(__uint_as_float((uint32_t)(c >> 32))) << 32) | (uint32_t)c;
    }
    __syncthreads();
  }

  // Ranks: each candidate counts the candidates of its segment ahead of it.
  const int64_t ob = row * K;
  for (uint32_t i = (uint32_t)t; i < nc; i += (uint32_t)stride) {
    const uint64_t mine = lds.cand[i];
    const uint32_t id = 0xffffffffu - (uint32_t)mine;
    // Loaded ahead of the count, which then covers its latency; every
    // candidate's id lies in the valid prefix, so below NB.
    const int32_t page = g.page_table[(int64_t)b * g.NB + (id < (uint32_t)g.NB ? id : 0u)];
    uint32_t st = 0, len = nc;
    if (!refine) {
      const uint32_t bb = degen ? 1u : fbin(key_score((uint32_t)(mine >> 32)), s, c);
      len = lds.hist[bb];
      st = (lds.above[bb] >> 3) - len;   // the scatter advanced the cursor by 8 per entry
    }
    st = st < nc ? st : nc;
    const uint32_t end = len < nc - st ? st + len : nc;
    uint32_t r = st;
    for (uint32_t j = st; j < end; j += 4) {     // reads stay inside cand[CAP + 4]
      const uint64_t c0 = lds.cand[j], c1 = lds.cand[j + 1], c2 = lds.cand[j + 2], c3 = lds.cand[j + 3];
      r += (c0 > mine ? 1u : 0u) + (j + 1 < end && c1 > mine ? 1u : 0u) +
           (j + 2 < end && c2 > mine ? 1u : 0u) + (j + 3 < end && c3 > mine ? 1u : 0u);
    }
    if (r < (uint32_t)K && id < (uint32_t)g.NB) {
      g.out_blocks[ob + r] = (int32_t)id;
      g.out_pages[ob + r] = page;
    }
  }
  for (int i = (int)nc + t; i < K; i += stride) {
    g.out_blocks[ob + i] = -1;
    g.out_pages[ob + i] = -1;
  }
}

bool aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }

// Multiplier and shifts of unsigned division by d (1 <= d < 2^31) for
// dividends below 2^32: l = ceil(log2 d), m = floor(2^32 (2^l - d) / d) + 1
// (Granlund and Montgomery, "Division by invariant integers using
// multiplication", 1994, section 4).
void set_divisor(DArgs& g, uint32_t d) {
  uint32_t l = 0;
  while ((1ull << l) < d) ++l;
  g.bs_mul = (uint32_t)(((1ull << 32) * ((1ull << l) - d)) / d + 1);
  g.bs_sh1 = l < 1 ? l : 1;
  g.bs_sh2 = l > 1 ? l - 1 : 0;
}

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
  const int64_t chunks = (NB + kChunk - 1) / kChunk;
  const int waves = (int)(chunks < kMaxWaves ? chunks : kMaxWaves);
  // Q workgroups of 64 * waves work-items along grid x: fewer than 2^32.
  if (rows > (int64_t)INT32_MAX || H > kMaxGridYZ || B > kMaxGridYZ ||
      Q * 64 * waves >= (1ll << 32))
    return FAGQ_E_TOO_LARGE;
  if (!aligned(scores, (uintptr_t)esz) || !aligned(page_table, 4) || !aligned(out_blocks, 4) ||
      !aligned(out_pages, 4) || !aligned(q_pos, index_dtype == FAGQ_DSA_I64 ? 8 : 4) ||
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
  set_divisor(g, (uint32_t)block_size);
  // 16-byte vector loads need every row 16-byte aligned; rows of more than
  // kMaxWaves chunks are walked chunk by chunk.
  const int bf16 = scores_dtype == FAGQ_DSA_BF16;
  const int vec = aligned(scores, 16) && (NB * esz) % 16 == 0;
  const int kind = chunks > kMaxWaves ? kLongRows : chunks > kSmallWaves ? kRows : kSmallRows;
  const int large = top_k > kSmallTopK;
#define FAGQ_DSA_C(B, V, KIND) \
  {(const void*)&dsa_topk_rows<B, V, KIND, kCapSmall>, \
   (const void*)&dsa_topk_rows<B, V, KIND, kCapLarge>}
#define FAGQ_DSA_K(B, V) \
  {FAGQ_DSA_C(B, V, kSmallRows), FAGQ_DSA_C(B, V, kRows), FAGQ_DSA_C(B, V, kLongRows)}
  static const void* const kernels[2][2][3][2] = {
      {FAGQ_DSA_K(false, false), FAGQ_DSA_K(false, true)},
      {FAGQ_DSA_K(true, false), FAGQ_DSA_K(true, true)}};
#undef FAGQ_DSA_K
#undef FAGQ_DSA_C
  void* args[] = {&g};
  return launch_kernel(kernels[bf16][vec][kind][large], dim3((unsigned)Q, (unsigned)H, (unsigned)B),
                       dim3((unsigned)(64 * waves)), args, 0, static_cast<hipStream_t>(stream));
}

}  // extern "C"
