// fagq_dispatch.hpp - the library's one kernel-launch wrapper, and the launch
// lookups shared by the instantiation units and the C ABI.  One lookup per
// (code format, scale format), indexed by the lanes-per-group index, the steps
// per wave, whether norm_out is written and the row-group mode.
#pragma once

#include <hip/hip_runtime.h>

#include "fagq_kernels.hpp"

namespace fagq {

// (args, grid, block, dynamic LDS bytes, stream) -> launch_kernel's status
using LaunchFn = int (*)(const KArgs&, dim3, dim3, unsigned, hipStream_t);
using PartsLaunchFn = int (*)(const PArgs&, dim3, dim3, unsigned, hipStream_t);

constexpr int kNumLpg = 3;      // lanes per group 8, 16, 32  <->  G = 64, 128, 256

constexpr int lpg_index(int group_size) {
  return group_size == 64 ? 0 : group_size == 128 ? 1 : group_size == 256 ? 2 : -1;
}


// FAGQ_OK if the current device is gfx950 (cached per device), else
// FAGQ_E_DEVICE or -hipError_t.
int device_check();

// Every kernel launch of the library goes through launch_kernel; its status
// is 0 (FAGQ_OK) or -hipError_t.  Built with -DFAGQ_TEST_LAUNCH_FAILURE (a
// test build only, never the shipped library) it launches nothing and reports
// hipErrorLaunchFailure, so that CPU tests can check how a launch failure
// propagates through the C ABI without any kernel reaching a device.
inline int launch_kernel(const void* fn, dim3 grid, dim3 block, void** args, size_t lds,
                         hipStream_t stream) {
#ifdef FAGQ_TEST_LAUNCH_FAILURE
  (void)fn, (void)grid, (void)block, (void)args, (void)lds, (void)stream;
  return -(int)hipErrorLaunchFailure;
#else
  const hipError_t e = hipLaunchKernel(fn, grid, block, args, lds, stream);
  return e == hipSuccess ? 0 : -(int)e;
#endif
}

// lookup_q<code>_s<scale>(lpg index, steps per wave in [1, 4], norm, row-group mode).
LaunchFn lookup_q0_s0(int lpg_idx, int steps, bool norm, int mode);   // fp8, f32
LaunchFn lookup_q0_s1(int lpg_idx, int steps, bool norm, int mode);   // fp8, ue8m0
LaunchFn lookup_q1_s0(int lpg_idx, int steps, bool norm, int mode);   // int8 rne, f32
LaunchFn lookup_q1_s1(int lpg_idx, int steps, bool norm, int mode);   // int8 rne, ue8m0
LaunchFn lookup_q2_s0(int lpg_idx, int steps, bool norm, int mode);   // int8 trunc, f32
LaunchFn lookup_q2_s1(int lpg_idx, int steps, bool norm, int mode);   // int8 trunc, ue8m0

// Typed form, fp16 tensors (fagq_rows with ET_F16): lookup_f16_q<code>_s<scale>(lpg
// index, steps per wave in [1, 4], norm, row-group mode).
LaunchFn lookup_f16_q0_s0(int lpg_idx, int steps, bool norm, int mode);
LaunchFn lookup_f16_q0_s1(int lpg_idx, int steps, bool norm, int mode);
LaunchFn lookup_f16_q1_s0(int lpg_idx, int steps, bool norm, int mode);
LaunchFn lookup_f16_q1_s1(int lpg_idx, int steps, bool norm, int mode);
LaunchFn lookup_f16_q2_s0(int lpg_idx, int steps, bool norm, int mode);
LaunchFn lookup_f16_q2_s1(int lpg_idx, int steps, bool norm, int mode);

// Typed form, families with an fp32 tensor (fagq_rows_typed):
// lookup_typed_q<code>_s<scale>(lpg index, steps per wave in [1, 4], norm, type
// family in [TF_BF16_R32, TF_F32]).
LaunchFn lookup_typed_q0_s0(int lpg_idx, int steps, bool norm, int family);
LaunchFn lookup_typed_q0_s1(int lpg_idx, int steps, bool norm, int family);
LaunchFn lookup_typed_q1_s0(int lpg_idx, int steps, bool norm, int family);
LaunchFn lookup_typed_q1_s1(int lpg_idx, int steps, bool norm, int family);
LaunchFn lookup_typed_q2_s0(int lpg_idx, int steps, bool norm, int family);
LaunchFn lookup_typed_q2_s1(int lpg_idx, int steps, bool norm, int family);

// Multi-input form (fagq_rows_parts): lookup_parts_q<code>_s<scale>(lpg index,
// steps per wave 1, 2 or 4).
PartsLaunchFn lookup_parts_q0_s0(int lpg_idx, int steps);
PartsLaunchFn lookup_parts_q0_s1(int lpg_idx, int steps);
PartsLaunchFn lookup_parts_q1_s0(int lpg_idx, int steps);
PartsLaunchFn lookup_parts_q1_s1(int lpg_idx, int steps);
PartsLaunchFn lookup_parts_q2_s0(int lpg_idx, int steps);
PartsLaunchFn lookup_parts_q2_s1(int lpg_idx, int steps);

}  // namespace fagq
