// fagq_dispatch.hpp - launch lookups shared by the instantiation units and the
// C ABI.  One lookup per (code format, scale format), indexed by the
// lanes-per-group index, the steps per wave, whether norm_out is written and
// the rows-in-sequence index.
#pragma once

#include <hip/hip_runtime.h>

#include "fagq_kernels.hpp"

namespace fagq {

// (args, grid, block, dynamic LDS bytes, stream)
using LaunchFn = hipError_t (*)(const KArgs&, dim3, dim3, unsigned, hipStream_t);
using PartsLaunchFn = hipError_t (*)(const PArgs&, dim3, dim3, unsigned, hipStream_t);

constexpr int kNumLpg = 3;      // lanes per group 8, 16, 32  <->  G = 64, 128, 256

constexpr int lpg_index(int group_size) {
  return group_size == 64 ? 0 : group_size == 128 ? 1 : group_size == 256 ? 2 : -1;
}


// FAGQ_OK if the current device is gfx950 (cached per device), else
// FAGQ_E_DEVICE or -hipError_t.
int device_check();

// Status of a kernel launch: 0 (FAGQ_OK) or -hipError_t.  Built with
// -DFAGQ_TEST_LAUNCH_FAILURE (a test build only, never the shipped library)
// every launch reports hipErrorLaunchFailure instead, so that the CPU tests
// can check how a launch failure propagates through the C ABI.
#ifdef FAGQ_TEST_LAUNCH_FAILURE
inline int launch_status(hipError_t) { return -(int)hipErrorLaunchFailure; }
#else
inline int launch_status(hipError_t e) { return e == hipSuccess ? 0 : -(int)e; }
#endif

// lookup_q<code>_s<scale>(lpg index, steps per wave in [1, 4], norm, row-group mode).
LaunchFn lookup_q0_s0(int lpg_idx, int steps, bool norm, int mode);   // fp8, f32
LaunchFn lookup_q0_s1(int lpg_idx, int steps, bool norm, int mode);   // fp8, ue8m0
LaunchFn lookup_q1_s0(int lpg_idx, int steps, bool norm, int mode);   // int8 rne, f32
LaunchFn lookup_q1_s1(int lpg_idx, int steps, bool norm, int mode);   // int8 rne, ue8m0
LaunchFn lookup_q2_s0(int lpg_idx, int steps, bool norm, int mode);   // int8 trunc, f32
LaunchFn lookup_q2_s1(int lpg_idx, int steps, bool norm, int mode);   // int8 trunc, ue8m0

// Multi-input form (fagq_rows_parts): lookup_parts_q<code>_s<scale>(lpg index,
// steps per wave in [1, kMaxStepsParts]).
PartsLaunchFn lookup_parts_q0_s0(int lpg_idx, int steps);
PartsLaunchFn lookup_parts_q0_s1(int lpg_idx, int steps);
PartsLaunchFn lookup_parts_q1_s0(int lpg_idx, int steps);
PartsLaunchFn lookup_parts_q1_s1(int lpg_idx, int steps);
PartsLaunchFn lookup_parts_q2_s0(int lpg_idx, int steps);
PartsLaunchFn lookup_parts_q2_s1(int lpg_idx, int steps);

}  // namespace fagq
