// fagq_probe.hip - measurement probes (libfagq_probe.so, include/fagq_probe.h):
// the HBM streams with the operator's cache policies (the achievable-bandwidth
// ceilings and the byte-counter calibration), the fp8 GEMM's matrix
// instruction issued from registers, and the LDS read patterns of the GEMM's
// operand tiles.  They measure the machine the operators run on and are not
// part of the drop-in library (libfagq.so).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "fagq.h"
#include "fagq_dispatch.hpp"
#include "fagq_gemm_lds.hpp"
#include "fagq_probe.h"

namespace fagq {
namespace probe {
namespace {

using gemm::kBK;
using gemm::swz;
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

bool aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }

// HBM ceiling probes (and byte-counter calibration): every thread moves one
// 16-byte chunk through buffer descriptors, with the operator's cache
// policies (non-temporal loads, sc1 | nt stores).  kStreamBlock threads per
// workgroup, one workgroup per kStreamBlock * 16 bytes.
constexpr int kStreamBlock = 512;

__device__ __forceinline__ uint32_t chunk_bytes(int64_t bytes) {
  const int64_t rem = bytes - (int64_t)blockIdx.x * kStreamBlock * 16;
  return rem > kStreamBlock * 16 ? kStreamBlock * 16u : (uint32_t)rem;
}

__global__ void __launch_bounds__(kStreamBlock) fagq_stream_copy(const uint8_t* src, uint8_t* dst,
                                                                 int64_t bytes) {
  const int64_t base = (int64_t)blockIdx.x * kStreamBlock * 16;
  const uint32_t n = chunk_bytes(bytes);
  const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(make_rsrc(src + base, n), threadIdx.x * 16,
                                                        0, kNonTemporal);
  __builtin_amdgcn_raw_buffer_store_b128(v, make_rsrc(dst + base, n), threadIdx.x * 16, 0,
                                         kStoreAux);
}

// Read-only: the loaded data is kept live by a store to dst[0..15] that runs
// only when a chunk's four words XOR to 0x9e3779b9.
__global__ void __launch_bounds__(kStreamBlock) fagq_stream_read(const uint8_t* src, uint8_t* dst,
                                                                 int64_t bytes) {
  const int64_t base = (int64_t)blockIdx.x * kStreamBlock * 16;
  const uint32_t n = chunk_bytes(bytes);
  const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(make_rsrc(src + base, n), threadIdx.x * 16,
                                                        0, kNonTemporal);
  if ((v[0] ^ v[1] ^ v[2] ^ v[3]) == 0x9e3779b9u)
    __builtin_amdgcn_raw_buffer_store_b128(v, make_rsrc(dst, 16), 0, 0, 0);
}

// Write-only: each chunk gets (its byte offset, thread, 2, 3).
__global__ void __launch_bounds__(kStreamBlock) fagq_stream_write(const uint8_t*, uint8_t* dst,
                                                                  int64_t bytes) {
  const int64_t base = (int64_t)blockIdx.x * kStreamBlock * 16;
  const uint32_t n = chunk_bytes(bytes);
  const u32x4 v = {(uint32_t)base, threadIdx.x, 2u, 3u};
  __builtin_amdgcn_raw_buffer_store_b128(v, make_rsrc(dst + base, n), threadIdx.x * 16, 0,
                                         kStoreAux);
}

// The operator's byte mix without its arithmetic: every thread reads 16
// bytes of x and of residual (8 bf16 each) and writes 16 bytes of
// residual_out and 8 bytes of codes.  x, residual = src, src + bytes;
// residual_out, codes = dst, dst + bytes.
__global__ void __launch_bounds__(kStreamBlock) fagq_stream_opmix(const uint8_t* src, uint8_t* dst,
                                                                  int64_t bytes) {
  const int64_t base = (int64_t)blockIdx.x * kStreamBlock * 16;
  const uint32_t n = chunk_bytes(bytes);
  const u32x4 x = __builtin_amdgcn_raw_buffer_load_b128(make_rsrc(src + base, n), threadIdx.x * 16,
                                                        0, kNonTemporal);
  const u32x4 r = __builtin_amdgcn_raw_buffer_load_b128(make_rsrc(src + bytes + base, n),
                                                        threadIdx.x * 16, 0, kNonTemporal);
  const u32x4 s = x ^ r;
  __builtin_amdgcn_raw_buffer_store_b128(s, make_rsrc(dst + base, n), threadIdx.x * 16, 0,
                                         kStoreAux);
  __builtin_amdgcn_raw_buffer_store_b64(u32x2{s[0] ^ s[1], s[2] ^ s[3]},
                                        make_rsrc(dst + bytes + base / 2, n / 2), threadIdx.x * 8,
                                        0, kStoreAux);
}

// Issue-rate probe of the GEMM's instruction: every wave keeps 8 independent
// 16 x 16 accumulators and issues iters x 8 v_mfma_scale_f32_16x16x128_f8f6f4
// (E8M0 scales 2^-7 and 2^3) on register operands, with no memory access in
// the loop; each thread then writes the sum of its accumulators.
constexpr int kPeakThreads = 256;
constexpr int kPeakChain = 8;
__global__ void __launch_bounds__(kPeakThreads) mfma_peak_kernel(float* out, int iters) {
  const int t = threadIdx.x;
  i32x8 a, b;
#pragma unroll
  for (int i = 0; i < 8; ++i) {   // fp8 e4m3 values near 1.0 (0x38) and 0.5 (0x30)
    a[i] = 0x38383838 ^ (t * 7 + i);
    b[i] = 0x30303030 ^ (t * 3 + i);
  }
  f32x4 c[kPeakChain] = {};
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int j = 0; j < kPeakChain; ++j)
      c[j] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c[j], 0, 0, 0, 120, 0, 130);
  }
  float r = 0.0f;
#pragma unroll
  for (int j = 0; j < kPeakChain; ++j) r += c[j][0] + c[j][1] + c[j][2] + c[j][3];
  out[(int64_t)blockIdx.x * kPeakThreads + t] = r;
}

// The 32 x 32 x 64 shape: every wave keeps 4 independent 32 x 32
// accumulators (16 floats per lane each) and issues iters x 4 instructions,
// each twice the flops of one 16 x 16 x 128.
typedef float f32x16 __attribute__((ext_vector_type(16)));
constexpr int kPeakChain32 = 4;
__global__ void __launch_bounds__(kPeakThreads) mfma_peak32_kernel(float* out, int iters) {
  const int t = threadIdx.x;
  i32x8 a, b;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    a[i] = 0x38383838 ^ (t * 7 + i);
    b[i] = 0x30303030 ^ (t * 3 + i);
  }
  f32x16 c[kPeakChain32] = {};
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int j = 0; j < kPeakChain32; ++j)
      c[j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c[j], 0, 0, 0, 120, 0, 130);
  }
  float r = 0.0f;
#pragma unroll
  for (int j = 0; j < kPeakChain32; ++j)
#pragma unroll
    for (int i = 0; i < 16; ++i) r += c[j][i];
  out[(int64_t)blockIdx.x * kPeakThreads + t] = r;
}

// LDS bank probe.  Every lane of 4 waves reads the 16 bytes at
// lds_probe_addr(pattern, lane % 64) with ds_read_b128, 8 x iters times, from 16
// KB of LDS holding word i = i * 0x9E3779B1, then writes the 4 words it read.
// Patterns 1-5 are one MFMA operand fragment of a 16-row tile of 128-byte
// rows: lane l reads row l % 16 at logical chunk 2 (l / 16) (pattern 2: the
// chunk after it).
constexpr int kLdsProbeThreads = 256;
constexpr int kLdsProbeWords = 4096;
__device__ __forceinline__ int lds_probe_addr(int pattern, int lane) {
  const int r = lane & 15, c = (lane >> 4) * 2 + (pattern == 2 ? 1 : 0);
  switch (pattern) {
    case 0: return lane * 16;                                 // 1 KB in lane order
    case 1:
    case 2: return r * kBK + (swz(c, r) << 4);                // the GEMM's swizzle
    case 3: return r * kBK + ((c ^ ((r >> 1) & 7)) << 4);     // chunk c ^ ((r / 2) % 8)
    case 4: return r * kBK + ((c ^ (r & 7)) << 4);            // chunk c ^ (r % 8)
    default: return r * kBK + (c << 4);                       // no swizzle
  }
}

__global__ void __launch_bounds__(kLdsProbeThreads) lds_probe_kernel(int32_t* out, int pattern,
                                                                     int iters) {
  __shared__ __attribute__((aligned(1024))) int32_t words[kLdsProbeWords];
  for (int i = threadIdx.x; i < kLdsProbeWords; i += kLdsProbeThreads)
    words[i] = (int32_t)((uint32_t)i * 0x9E3779B1u);
  __syncthreads();
  const uint32_t a = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) int32_t*)words +
                     (uint32_t)lds_probe_addr(pattern, threadIdx.x & 63);
  i32x4 v = {0, 0, 0, 0};
  for (int it = 0; it < iters; ++it) {
    i32x4 v0, v1, v2, v3, v4, v5, v6, v7;
    asm volatile(
        "ds_read_b128 %0, %8\n\t"
        "ds_read_b128 %1, %8\n\t"
        "ds_read_b128 %2, %8\n\t"
        "ds_read_b128 %3, %8\n\t"
        "ds_read_b128 %4, %8\n\t"
        "ds_read_b128 %5, %8\n\t"
        "ds_read_b128 %6, %8\n\t"
        "ds_read_b128 %7, %8\n\t"
        "s_waitcnt lgkmcnt(0)"
        : "=v"(v0), "=v"(v1), "=v"(v2), "=v"(v3), "=v"(v4), "=v"(v5), "=v"(v6), "=v"(v7)
        : "v"(a));
    v = v0 & v1 & v2 & v3 & v4 & v5 & v6 & v7;   // all eight read the same bytes
  }
  i32x4* o = reinterpret_cast<i32x4*>(out) + (int64_t)blockIdx.x * kLdsProbeThreads + threadIdx.x;
  *o = v;
}

}  // namespace
}  // namespace probe
}  // namespace fagq

using namespace fagq;
using namespace fagq::probe;

extern "C" {

FAGQ_API int fagq_diag_stream(const void* src, void* dst, int64_t bytes, int mode,
                              void* stream) {
  if (mode < FAGQ_STREAM_COPY || mode > FAGQ_STREAM_OPMIX) return FAGQ_E_FORMAT;
  if ((mode != FAGQ_STREAM_WRITE && !src) || !dst) return FAGQ_E_NULL;
  if (bytes < 0 || bytes % (mode == FAGQ_STREAM_OPMIX ? 32 : 16) != 0) return FAGQ_E_SHAPE;
  if ((src && !aligned(src, 16)) || !aligned(dst, 16)) return FAGQ_E_ALIGN;
  if (bytes == 0) return FAGQ_OK;
  const int64_t blocks = (bytes + kStreamBlock * 16 - 1) / (kStreamBlock * 16);
  if (blocks > INT32_MAX) return FAGQ_E_TOO_LARGE;
  const int dc = device_check();
  if (dc != FAGQ_OK) return dc;
  const uint8_t* s8 = static_cast<const uint8_t*>(src);
  uint8_t* d8 = static_cast<uint8_t*>(dst);
  int64_t n = bytes;
  void* args[] = {&s8, &d8, &n};
  const void* k = mode == FAGQ_STREAM_COPY    ? reinterpret_cast<const void*>(&fagq_stream_copy)
                  : mode == FAGQ_STREAM_READ  ? reinterpret_cast<const void*>(&fagq_stream_read)
                  : mode == FAGQ_STREAM_WRITE ? reinterpret_cast<const void*>(&fagq_stream_write)
                                              : reinterpret_cast<const void*>(&fagq_stream_opmix);
  return launch_kernel(k, dim3((unsigned)blocks), dim3(kStreamBlock), args, 0,
                       static_cast<hipStream_t>(stream));
}

FAGQ_API int fagq_diag_copy(const void* src, void* dst, int64_t bytes, void* stream) {
  return fagq_diag_stream(src, dst, bytes, FAGQ_STREAM_COPY, stream);
}

FAGQ_API int fagq_diag_mfma_peak(float* out, int64_t blocks, int32_t iters, void* stream) {
  return fagq_diag_mfma_rate(out, blocks, iters, 0, stream);
}

FAGQ_API int fagq_diag_lds_read(int32_t* out, int64_t blocks, int32_t iters, int pattern,
                                void* stream) {
  if (!out) return FAGQ_E_NULL;
  if (pattern < 0 || pattern > 5) return FAGQ_E_FORMAT;
  if (blocks < 1 || iters < 1) return FAGQ_E_SHAPE;
  if (blocks > (1 << 20) || iters > (1 << 20)) return FAGQ_E_TOO_LARGE;
  if (!aligned(out, 16)) return FAGQ_E_ALIGN;
  const int dc = device_check();
  if (dc != FAGQ_OK) return dc;
  int pt = pattern, it = iters;
  void* args[] = {&out, &pt, &it};
  return launch_kernel(reinterpret_cast<const void*>(&lds_probe_kernel), dim3((unsigned)blocks),
                       dim3(kLdsProbeThreads), args, 0, static_cast<hipStream_t>(stream));
}

FAGQ_API int fagq_diag_mfma_rate(float* out, int64_t blocks, int32_t iters, int shape,
                                 void* stream) {
  if (!out) return FAGQ_E_NULL;
  if (shape != 0 && shape != 1) return FAGQ_E_FORMAT;
  if (blocks < 1 || iters < 1) return FAGQ_E_SHAPE;
  if (blocks > (1 << 20) || iters > (1 << 20)) return FAGQ_E_TOO_LARGE;
  if (!aligned(out, 4)) return FAGQ_E_ALIGN;
  const int dc = device_check();
  if (dc != FAGQ_OK) return dc;
  int it = iters;
  void* args[] = {&out, &it};
  const void* k = shape == 0 ? reinterpret_cast<const void*>(&mfma_peak_kernel)
                             : reinterpret_cast<const void*>(&mfma_peak32_kernel);
  return launch_kernel(k, dim3((unsigned)blocks), dim3(kPeakThreads), args, 0,
                       static_cast<hipStream_t>(stream));
}

}  // extern "C"
