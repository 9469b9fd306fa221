// fagq_inst.hip - instantiates fagq_rows for one (code format, scale format)
// pair, selected with -DFAGQ_QF=<0|1|2> -DFAGQ_SF=<0|1>, for every supported
// group size and every steps-per-wave count, and exports its launch lookup.
#include "fagq_dispatch.hpp"

#ifndef FAGQ_QF
#error "FAGQ_QF must be defined"
#endif
#ifndef FAGQ_SF
#error "FAGQ_SF must be defined"
#endif

#define FAGQ_CAT4(a, b, c, d) a##b##c##d
#define FAGQ_LOOKUP(q, s) FAGQ_CAT4(lookup_q, q, _s, s)

namespace fagq {
namespace {

template <int NS, int LPG>
hipError_t launch_rows(const KArgs& a, dim3 grid, dim3 block, hipStream_t stream) {
  void* args[] = {const_cast<KArgs*>(&a)};
  return hipLaunchKernel(reinterpret_cast<const void*>(&fagq_rows<NS, LPG, FAGQ_QF, FAGQ_SF>),
                         grid, block, args, 0, stream);
}

}  // namespace

#define FAGQ_ROW(LPG)                                                                          \
  {&launch_rows<1, LPG>,  &launch_rows<2, LPG>,  &launch_rows<3, LPG>,  &launch_rows<4, LPG>,  \
   &launch_rows<5, LPG>,  &launch_rows<6, LPG>,  &launch_rows<7, LPG>,  &launch_rows<8, LPG>,  \
   &launch_rows<9, LPG>,  &launch_rows<10, LPG>, &launch_rows<11, LPG>, &launch_rows<12, LPG>, \
   &launch_rows<13, LPG>, &launch_rows<14, LPG>, &launch_rows<15, LPG>, &launch_rows<16, LPG>}

static_assert(kMaxStepsPerWave == 16, "FAGQ_ROW lists 16 step counts");

// The table lives in a host function so that device compilation never sees
// pointers to host launch stubs.
LaunchFn FAGQ_LOOKUP(FAGQ_QF, FAGQ_SF)(int lpg_idx, int steps) {
  static const LaunchFn table[kNumLpg][kMaxStepsPerWave] = {FAGQ_ROW(8), FAGQ_ROW(16), FAGQ_ROW(32)};
  return table[lpg_idx][steps - 1];
}

}  // namespace fagq
