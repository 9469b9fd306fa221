// fagq_inst_typed.hip - instantiates fagq_rows_typed for one (code format,
// scale format) pair, selected with -DFAGQ_QF=<0|1|2> -DFAGQ_SF=<0|1>, for
// every group size, steps per wave, norm_out choice and type family, and
// exports its launch lookup.
#include "fagq_dispatch.hpp"

#ifndef FAGQ_QF
#error "FAGQ_QF must be defined"
#endif
#ifndef FAGQ_SF
#error "FAGQ_SF must be defined"
#endif

#define FAGQ_CAT4(a, b, c, d) a##b##c##d
#define FAGQ_LOOKUP_TYPED(q, s) FAGQ_CAT4(lookup_typed_q, q, _s, s)

namespace fagq {
namespace {

template <int NS, int LPG, bool NORM, int TF>
int launch_typed(const KArgs& a, dim3 grid, dim3 block, unsigned lds, hipStream_t stream) {
  void* args[] = {const_cast<KArgs*>(&a)};
  return launch_kernel(
      reinterpret_cast<const void*>(&fagq_rows_typed<NS, LPG, FAGQ_QF, FAGQ_SF, NORM, TF>), grid,
      block, args, lds, stream);
}

}  // namespace

#define FAGQ_T(NS, LPG, NORM) \
  {&launch_typed<NS, LPG, NORM, TF_F16>, &launch_typed<NS, LPG, NORM, TF_BF16_R32>, \
   &launch_typed<NS, LPG, NORM, TF_F16_R32>, &launch_typed<NS, LPG, NORM, TF_F32>}
#define FAGQ_TN(NS, LPG) {FAGQ_T(NS, LPG, false), FAGQ_T(NS, LPG, true)}
#define FAGQ_TS(LPG) {FAGQ_TN(1, LPG), FAGQ_TN(2, LPG), FAGQ_TN(3, LPG), FAGQ_TN(4, LPG)}

static_assert(kMaxStepsPerWave == 4, "FAGQ_TS lists 4 step counts");
static_assert(kNumTypeFamilies == 4, "FAGQ_T lists 4 type families");

LaunchFn FAGQ_LOOKUP_TYPED(FAGQ_QF, FAGQ_SF)(int lpg_idx, int steps, bool norm, int family) {
  static const LaunchFn table[kNumLpg][kMaxStepsPerWave][2][kNumTypeFamilies] = {
      FAGQ_TS(8), FAGQ_TS(16), FAGQ_TS(32)};
  return table[lpg_idx][steps - 1][norm ? 1 : 0][family];
}

}  // namespace fagq
