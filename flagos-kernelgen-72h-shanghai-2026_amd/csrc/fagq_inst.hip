// fagq_inst.hip - instantiates fagq_rows for one (code format, scale format)
// pair, selected with -DFAGQ_QF=<0|1|2> -DFAGQ_SF=<0|1>, for every supported
// group size, steps per wave, norm_out choice and row-group mode,
// and fagq_rows_parts for every group size and steps per wave, and exports
// their launch lookups.
#include "fagq_dispatch.hpp"

#ifndef FAGQ_QF
#error "FAGQ_QF must be defined"
#endif
#ifndef FAGQ_SF
#error "FAGQ_SF must be defined"
#endif

#define FAGQ_CAT4(a, b, c, d) a##b##c##d
#define FAGQ_LOOKUP(q, s) FAGQ_CAT4(lookup_q, q, _s, s)
#define FAGQ_LOOKUP_PARTS(q, s) FAGQ_CAT4(lookup_parts_q, q, _s, s)

namespace fagq {
namespace {

template <int NS, int LPG, bool NORM, int MODE>
int launch_rows(const KArgs& a, dim3 grid, dim3 block, unsigned lds, hipStream_t stream) {
  void* args[] = {const_cast<KArgs*>(&a)};
  return launch_kernel(
      reinterpret_cast<const void*>(&fagq_rows<NS, LPG, FAGQ_QF, FAGQ_SF, NORM, MODE>), grid,
      block, args, lds, stream);
}

template <int NS, int LPG>
int launch_rows_parts(const PArgs& a, dim3 grid, dim3 block, unsigned lds,
                      hipStream_t stream) {
  void* args[] = {const_cast<PArgs*>(&a)};
  return launch_kernel(
      reinterpret_cast<const void*>(&fagq_rows_parts<NS, LPG, FAGQ_QF, FAGQ_SF>), grid, block,
      args, lds, stream);
}

}  // namespace

#define FAGQ_R(NS, LPG, NORM) \
  {&launch_rows<NS, LPG, NORM, RG_INDEPENDENT>, &launch_rows<NS, LPG, NORM, RG_SHARED_GAMMA>, \
   &launch_rows<NS, LPG, NORM, RG_WIDE_SCALES>}
#define FAGQ_N(NS, LPG) {FAGQ_R(NS, LPG, false), FAGQ_R(NS, LPG, true)}
#define FAGQ_S(LPG) {FAGQ_N(1, LPG), FAGQ_N(2, LPG), FAGQ_N(3, LPG), FAGQ_N(4, LPG)}

static_assert(kMaxStepsPerWave == 4, "FAGQ_S lists 4 step counts");
static_assert(kNumModes == 3, "FAGQ_R lists 3 row-group modes");

// The table lives in a host function so that device compilation never sees
// pointers to host launch stubs.
LaunchFn FAGQ_LOOKUP(FAGQ_QF, FAGQ_SF)(int lpg_idx, int steps, bool norm, int mode) {
  static const LaunchFn table[kNumLpg][kMaxStepsPerWave][2][kNumModes] = {
      FAGQ_S(8), FAGQ_S(16), FAGQ_S(32)};
  return table[lpg_idx][steps - 1][norm ? 1 : 0][mode];
}

static_assert(kMaxStepsParts == 4, "the parts table lists the step counts 1, 2 and 4");

// steps in {1, 2, 4} (the multi-input route never takes 3).
PartsLaunchFn FAGQ_LOOKUP_PARTS(FAGQ_QF, FAGQ_SF)(int lpg_idx, int steps) {
  static const PartsLaunchFn table[kNumLpg][3] = {
      {&launch_rows_parts<1, 8>, &launch_rows_parts<2, 8>, &launch_rows_parts<4, 8>},
      {&launch_rows_parts<1, 16>, &launch_rows_parts<2, 16>, &launch_rows_parts<4, 16>},
      {&launch_rows_parts<1, 32>, &launch_rows_parts<2, 32>, &launch_rows_parts<4, 32>}};
  return table[lpg_idx][steps == 4 ? 2 : steps - 1];
}

}  // namespace fagq
