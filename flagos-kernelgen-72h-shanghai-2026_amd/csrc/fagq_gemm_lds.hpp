// fagq_gemm_lds.hpp - the fp8 GEMM's LDS operand-tile layout, shared by the
// GEMM (fagq_gemm.hip) and the LDS bank probe that measures its reads
// (fagq_probe.hip).
#pragma once

#include <hip/hip_runtime.h>

namespace fagq {
namespace gemm {

constexpr int kBK = 128;   // k per block (one MFMA deep, one scale block): bytes per LDS tile row

// Position of logical 16-byte chunk c of LDS row r (only r % 8 matters).
__device__ __forceinline__ int swz_of(int r) { return ((r >> 1) & 1) | (r & 4); }
__device__ __forceinline__ int swz(int c, int r) { return c ^ swz_of(r); }

}  // namespace gemm
}  // namespace fagq
